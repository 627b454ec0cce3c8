"""Decode throughput of tinferno's token loop on one MI355X, at every workload of the
benchmark's configuration list.

Headline workload: the Llama-3.2-1B-shape Q8_0 synthetic GGUF (16 layers, d_model 2048, 32/8
heads, head_dim 64, FFN 8192, vocab 128256, tied lm_head, seed 42), a 6-token prompt from the
seed, greedy decode at batch 1, max-seq 512. A step is one decode token: embedding, 16 layers,
final norm, lm_head and the greedy argmax (Model::decode + sample_greedy).

    python bench.py [--gpus 1] [--steps 32] [--warmup 8] [--runs 5] [--no-cpu] [--quick]

Prints one JSON line. `value` is decode tok/s of K steps of the on-device greedy loop
(tf_hip_generate: one persistent step-kernel launch for the K steps, inputs resident in HBM),
timed between two synchronisations after W warm-up steps. `roofline` is that kernel's
achieved algorithmic GB/s (the K steps' bytes, Model::decode_bytes, over the HIP-event time
of the launch on the context's stream). `configs` holds every workload of the list, each
measured with bench_e2e's protocol (bench_e2e.cpp:38-59, 106-126): warm-up runs, then R runs
of once() -- reset, prefill (TTFT), n_predict x (greedy argmax on the device + decode), each
token one call -- reported as medians with IQR and per-token p50/p95/p99; next to it the
one-launch greedy loop over the same tokens gives the config's roofline object, and the
reference --stage v2 path (compiled from its own sources, oracle/_ref) on the host's cores
gives its cpu_baseline on the same workload (whole prompt, every token). `prefill` is the
512-token prompt on the matrix
cores (MFMA utilisation) and the prefill time by prompt length (2..1024 tokens),
`context_sweep` the decode rate after 512..4000-token prompts.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import tempfile
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X
COPY_CALIB_BYTES = 1 << 30
PUBLISHED_CPU_TOK_S = 10.74  # reference --stage v2, Llama-3.2-1B Q8_0, Ryzen 5 4600H 6c/12t (its published figure)
CPU_SHARE = 16  # host CPUs of one GPU's job on the GPU box (the box's worker-pool size)

# The workload list: (key, description, preset, prompt tokens, decode tokens, max-seq, KV layout)
CONFIGS = (
    ("cfg1", "Llama-3.2-1B-shape Q8_0, 6-token prompt, 32 greedy tokens, max-seq 512",
     "llama1b_q8", 6, 32, 512, 0),
    ("cfg2", "Qwen2.5-0.5B-shape Q8_0 + QKV bias, 16-token prompt, 128 greedy tokens",
     "qwen05b_q8", 16, 128, 512, 0),
    ("cfg3", "Llama-3.2-1B-shape mixed Q4_0 / Q4_1 (ffn_down of layers 0, 15) / Q6_K lm_head, 6-token prompt, "
             "64 greedy tokens", "llama1b_mixq4", 6, 64, 512, 0),
    ("cfg4", "Llama-3.2-1B-shape Q8_0, 512-token prompt, 16 greedy tokens", "llama1b_q8", 512, 16, 1024, 0),
    ("cfg5", "Qwen2.5-1.5B-shape Q8_0 + QKV bias, 4096-token prompt, head-major fp32 KV, max-seq 8192, "
             "256 greedy tokens", "qwen15b_q8", 4096, 256, 8192, 1),
)
HEADLINE = "cfg1"
# committed rocprofv3 --pmc summaries (FETCH_SIZE, WRITE_SIZE scaled by a known-size copy):
# HBM bytes per decoded token of the step kernel, per config
TRAFFIC_SUMMARIES = {
    "cfg1": ROOT / "profiles" / "decode_llama1b_q8_0_step_kernel_traffic.txt",
    "cfg2": ROOT / "profiles" / "decode_qwen05b_q8_0_step_kernel_traffic.txt",
    "cfg3": ROOT / "profiles" / "decode_llama1b_mixq4_step_kernel_traffic.txt",
    "cfg4": ROOT / "profiles" / "decode_llama1b_q8_0_512_step_kernel_traffic.txt",
    "cfg5": ROOT / "profiles" / "decode_qwen15b_q8_4096_step_kernel_traffic.txt",
}
# context sweep: decode after prompts of these lengths, cache of CTX_MAX_SEQ positions
CTX_PROMPTS = (512, 1024, 2048, 4000)
CTX_MAX_SEQ = 4096
CTX_STEPS = 16


# ---------------------------------------------------------------- statistics (bench_e2e.cpp:15-27)

def percentile(v, p):
    if not v:
        return 0.0
    v = sorted(v)
    idx = p * (len(v) - 1)
    i = int(idx)
    f = idx - i
    if i + 1 >= len(v):
        return v[-1]
    return v[i] * (1 - f) + v[i + 1] * f


def med_iqr(v, nd=3):
    return {"median": round(percentile(v, 0.5), nd), "q1": round(percentile(v, 0.25), nd),
            "q3": round(percentile(v, 0.75), nd)}


# ---------------------------------------------------------------- host facts

def host_cpus() -> dict:
    """Logical CPUs, physical cores, the affinity mask and the threads the CPU leg uses."""
    logical = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = logical
    cores = set()
    try:
        phys = core = None
        for line in open("/proc/cpuinfo"):
            if line.startswith("physical id"):
                phys = line.split(":")[1].strip()
            elif line.startswith("core id"):
                core = line.split(":")[1].strip()
            elif not line.strip():
                if core is not None:
                    cores.add((phys, core))
                phys = core = None
    except OSError:
        pass
    threads = max(1, min(CPU_SHARE, affinity))
    return {"hardware_concurrency": logical, "physical_cores": len(cores) or None, "affinity_cpus": affinity,
            "threads": threads, "pinned": False,
            "threads_note": f"reference v2 runs hardware_concurrency threads (main.cpp:79-81); the GPU box gives one "
                            f"GPU's job a {CPU_SHARE}-CPU share, so min(affinity, {CPU_SHARE}) threads, unpinned"}


def model_path(preset: str, seed: int) -> str:
    d = pathlib.Path(tempfile.gettempdir()) / "tinferno_bench"
    d.mkdir(parents=True, exist_ok=True)
    return str(d / f"{preset}-seed{seed}.gguf")


def ensure_model(pkg, preset: str, threads: int):
    info = pkg.synth_preset_info(preset)
    path = model_path(preset, info["seed"])
    if not os.path.exists(path):
        t0 = time.time()
        pkg.synth_write(preset, path, threads=threads)
        print(f"bench.py: wrote {path} in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    return path, info


def kernel_source_digest() -> str:
    """The kernel-source digest the counter summaries record (profsum.kernel_source_digest)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("profsum", ROOT / "agent-serve_amd" / "profsum.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.kernel_source_digest()


def measured_traffic(key: str, tokens: int, kernel: str):
    """HBM bytes of `tokens` decoded tokens of `kernel` from the config's committed counter
    summary, and where they come from: the summary, the commit and kernel-source digest it
    measured, and whether that digest is the one of the sources being benched (a summary of
    other sources is reported with current false and traffic null)."""
    path = TRAFFIC_SUMMARIES.get(key)
    per_token, meta = None, {}
    try:
        for line in path.read_text().splitlines():
            f = line.split()
            if len(f) == 3 and f[0] == "traffic_bytes_per_token" and f[1] == kernel:
                per_token = float(f[2])
            elif len(f) == 2 and f[0] in ("commit", "csrc_sha256"):
                meta[f[0]] = f[1]
    except (OSError, AttributeError):
        return None, None
    src = {"summary": os.path.relpath(path, ROOT), "commit": meta.get("commit"),
           "csrc_sha256": meta.get("csrc_sha256"),
           "current": meta.get("csrc_sha256") == kernel_source_digest()}
    if per_token is None or not src["current"]:
        return None, src
    return int(per_token * tokens), src


def prefill_flops(info, n):
    """Algorithmic FLOP of a prefill of n tokens: 2 per weight per token for the layer
    matrices, the causal attention (q.k and p.v over i + 1 positions for token i), and the
    lm_head of the last token."""
    D, F, L, H, G = info["n_embd"], info["n_ff"], info["n_layer"], info["n_head"], info["n_kv_head"]
    hd = D // H
    dense = 2.0 * n * L * (D * (H * hd + 2 * G * hd) + H * hd * D + 3 * D * F)
    attn = 4.0 * hd * (n * (n + 1) / 2) * H * L
    return dense + attn + 2.0 * D * info["n_vocab"], dense


# ---------------------------------------------------------------- the GPU legs

def e2e_once(m, prompt, n_predict):
    """bench_e2e's once() on the GPU: reset, prefill (its argmax is the first token), then
    n_predict x (decode of the current token; the call returns the next greedy argmax),
    every call synchronous. Returns (prefill_s, decode_s, per-token ms, ids)."""
    m.reset()
    t0 = time.perf_counter()
    _, tok = m.prefill(prompt, want_logits=False)
    prefill_s = time.perf_counter() - t0
    tok_ms, ids = [], []
    t0 = time.perf_counter()
    for _ in range(n_predict):
        u = time.perf_counter()
        ids.append(tok)
        _, tok = m.decode(tok, want_logits=False)
        tok_ms.append((time.perf_counter() - u) * 1e3)
    return prefill_s, time.perf_counter() - t0, tok_ms, ids


def gpu_config(pkg, key, desc, preset, n_prompt, n_dec, max_seq, layout, runs, warmup, threads):
    path, info = ensure_model(pkg, preset, threads)
    prompt = pkg.synth_prompt(info["seed"], n_prompt, info["n_vocab"])
    # load + upload: GGUF read, every tensor copied to the device and repacked (model.cpp:9-78)
    t0 = time.perf_counter()
    m = pkg.HipModel(path, max_seq=max_seq, kv_layout=layout)
    upload_s = time.perf_counter() - t0
    wall_first = None
    for w in range(max(1, warmup)):
        t0 = time.perf_counter()
        e2e_once(m, prompt, min(8, n_dec))
        if w == 0:
            wall_first = time.perf_counter() - t0
    pf_tps, dec_tps, ttft, p50, p95, p99, ids = [], [], [], [], [], [], None
    for _ in range(runs):
        ps, ds, tok_ms, ids = e2e_once(m, prompt, n_dec)
        pf_tps.append(n_prompt / ps)
        dec_tps.append(n_dec / ds)
        ttft.append(ps * 1e3)
        p50.append(percentile(tok_ms, 0.50))
        p95.append(percentile(tok_ms, 0.95))
        p99.append(percentile(tok_ms, 0.99))
    # the one-launch greedy loop over the same tokens: the roofline's kernel
    m.reset()
    m.prefill(prompt, want_logits=False)
    pf_dev_ms, _, _, pf_name = m.last_timing()
    t0 = time.perf_counter()
    gen = m.generate(n_dec)
    loop_wall = time.perf_counter() - t0
    k_ms, _, launches, k_name = m.last_timing()
    # the drop-in path: the reference's loop over the patched Model::decode, logits copied to
    # the host every step and sample_greedy there (bench_e2e.cpp:49-54)
    dropin_tps, dropin_ids = [], None
    for _ in range(max(1, runs // 2)):
        m.reset()
        logits, _ = m.prefill(prompt, want_logits=True)
        first = int(logits.argmax())
        t0 = time.perf_counter()
        dropin_ids = m.greedy_host(first, n_dec)
        dropin_tps.append(n_dec / (time.perf_counter() - t0))
    step_bytes = [m.decode_bytes(n_prompt + i) for i in range(n_dec)]
    achieved = sum(step_bytes) / (k_ms * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic(key, n_dec, k_name)
    path_name = "persistent step kernel" if m.decode_path() == m.PATH_STEP else "graph"
    m.close()
    return {
        "workload": desc,
        "prompt_tokens": n_prompt, "decode_tokens": n_dec, "max_seq": max_seq,
        "kv_cache": "fp32 " + ("head-major" if layout else "seq-major"),
        "decode_path": path_name, "prefill_path": pf_name,
        "runs": runs, "warmup": max(1, warmup),
        "e2e": {
            "decode_tok_s": med_iqr(dec_tps, 1), "prefill_tok_s": med_iqr(pf_tps, 1), "ttft_ms": med_iqr(ttft, 3),
            "decode_tok_ms_p50": round(statistics.median(p50), 4), "decode_tok_ms_p95": round(statistics.median(p95), 4),
            "decode_tok_ms_p99": round(statistics.median(p99), 4),
            "note": "one synchronous call per token (device argmax returned, no logits copy), host wall clock",
        },
        "dropin_loop": {"decode_tok_s": med_iqr(dropin_tps, 1),
                        "logits_bytes_per_token": 4 * info["n_vocab"],
                        "tokens_match_e2e": bool(list(dropin_ids) == list(ids)),
                        "note": "Model::decode as the backend patch forwards it: logits to the host every "
                                "token, first-max argmax on the host (C++ loop, tfh_greedy_host)"},
        "upload_s": round(upload_s, 3),
        "device_loop": {"decode_tok_s": round(n_dec / loop_wall, 1), "kernel_ms": round(k_ms, 4),
                        "launches": launches, "prefill_device_ms": round(pf_dev_ms, 4),
                        "prefill_tok_s": round(n_prompt / (pf_dev_ms * 1e-3), 1),
                        "tokens_match_e2e": bool(list(gen) == list(ids))},
        "bytes_per_step": round(statistics.mean(step_bytes)),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": k_name, "launches": launches,
                     "bytes_per_launch": round(sum(step_bytes) / launches),
                     "avg_launch_us": round(k_ms / launches * 1e3, 3)},
        "first_call_wall_s": round(wall_first, 3),
        "ids": [int(t) for t in gen],
    }


def prefill_run(pkg, preset, threads, n, reps):
    """Median device ms (HIP events around the call's kernels) and wall ms of `reps` prefills
    of the n-token prompt from a reset, after a first prompt that allocates the chunk buffers
    (its extra wall time is returned too)."""
    path, info = ensure_model(pkg, preset, threads)
    prompt = pkg.synth_prompt(info["seed"], n, info["n_vocab"])
    m = pkg.HipModel(path, max_seq=1024, kv_layout=0)
    t0 = time.perf_counter()
    m.prefill(prompt, want_logits=False)
    first_wall = time.perf_counter() - t0
    dev, wall = [], []
    for _ in range(reps):
        m.reset()
        t0 = time.perf_counter()
        m.prefill(prompt, want_logits=False)
        wall.append((time.perf_counter() - t0) * 1e3)
        dev.append(m.last_timing()[0])
    name = m.last_timing()[3]
    m.close()
    return info, name, statistics.median(dev), statistics.median(wall), first_wall * 1e3 - statistics.median(wall)


PF_LENGTHS = (2, 6, 16, 32, 64, 128, 256, 513, 1024)


def prefill_lengths(pkg, threads, reps=3):
    """Prefill time by prompt length on the Llama-3.2-1B shape (Q8_0, max-seq 2048): median
    device ms (HIP events) of `reps` prefills from a reset, after one of the same prompt."""
    path, info = ensure_model(pkg, "llama1b_q8", threads)
    m = pkg.HipModel(path, max_seq=2048, kv_layout=0)
    out = []
    for n in PF_LENGTHS:
        prompt = pkg.synth_prompt(info["seed"] + n, n, info["n_vocab"])
        m.reset()
        m.prefill(prompt, want_logits=False)
        dev = []
        for _ in range(reps):
            m.reset()
            m.prefill(prompt, want_logits=False)
            dev.append(m.last_timing()[0])
        d = statistics.median(dev)
        out.append({"tokens": n, "device_ms": round(d, 3), "tok_s": round(n / (d * 1e-3), 1)})
    m.close()
    return out


def prefill_leg(pkg, threads, reps=5):
    """The 512-token prompt of the Llama-3.2-1B shape on the matrix cores (Q8_0, and the
    Q4_0 / Q4_1 mix of the same shape), the layer matrices read in their HBM layout."""
    n = 512
    info, name, d_ms, w_ms, first_extra = prefill_run(pkg, "llama1b_q8", threads, n, reps)
    _, name4, d4_ms, w4_ms, _ = prefill_run(pkg, "llama1b_mixq4", threads, n, reps)
    flops, dense = prefill_flops(info, n)
    tflops = flops / (d_ms * 1e-3) / 1e12
    return {
        "workload": f"{n}-token prompt (uniform ids, seed {info['seed']}) of the Llama-3.2-1B shape, max-seq 1024",
        "path": name, "tokens": n, "device_ms": round(d_ms, 3), "wall_ms": round(w_ms, 3),
        "tok_s": round(n / (d_ms * 1e-3), 1), "tflop": round(flops / 1e12, 4), "dense_tflop": round(dense / 1e12, 4),
        "achieved_tflop_s": round(tflops, 2), "mfma_peak_tflop_s": MFMA_F16_PEAK_TFLOPS,
        "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "mfma_note": "algorithmic FLOP/s over the dense fp16 MFMA peak; the GEMMs issue two fp16 MFMAs "
                     "(activation hi and lo) per algorithmic product, attention three fp16 MFMAs per "
                     "product (fp16 operand pairs)",
        "first_prompt_extra_ms": round(first_extra, 1),
        "mixq4": {"path": name4, "device_ms": round(d4_ms, 3), "wall_ms": round(w4_ms, 3),
                  "tok_s": round(n / (d4_ms * 1e-3), 1),
                  "note": "the same prompt on the Q4_0 layer matrices (Q4_1 ffn_down in layers 0 and 15)"},
        "by_length": prefill_lengths(pkg, threads),
    }


def context_sweep(pkg, threads):
    """Decode rate by context length (the sweep the reference's roofline.py reads as bench
    "context" and its runs never produced): per prompt length, a prefill from a reset, then
    CTX_STEPS greedy tokens timed by HIP events; GB/s counts the weights once and the KV rows
    of every position read (Model::decode_bytes)."""
    path, info = ensure_model(pkg, "llama1b_q8", threads)
    m = pkg.HipModel(path, max_seq=CTX_MAX_SEQ, kv_layout=0)
    m.prefill(pkg.synth_prompt(info["seed"], 8, info["n_vocab"]), want_logits=False)
    m.generate(4)
    out = []
    for n in CTX_PROMPTS:
        prompt = pkg.synth_prompt(info["seed"] + n, n, info["n_vocab"])
        m.reset()
        m.prefill(prompt, want_logits=False)
        pf_ms = m.last_timing()[0]
        m.generate(CTX_STEPS)
        ms, _, _, name = m.last_timing()
        b = sum(m.decode_bytes(n + i) for i in range(CTX_STEPS))
        out.append({"context": n, "decode_tok_s": round(CTX_STEPS / (ms * 1e-3), 1),
                    "decode_gb_s": round(b / (ms * 1e-3) / 1e9, 1), "decode_path": name,
                    "kv_bytes_per_token": int(m.decode_bytes(n) - m.decode_bytes(0)),
                    "prefill_tok_s": round(n / (pf_ms * 1e-3), 1)})
    m.close()
    return {"max_seq": CTX_MAX_SEQ, "steps": CTX_STEPS, "points": out}


# ---------------------------------------------------------------- the CPU baselines

# the reference --stage v2 path per config: (prompt tokens, decode tokens, runs) — every
# workload whole; the Qwen2.5-1.5B shape's 4096-token prompt takes ≈ 85 s on 16 host threads
# (its prefill attention is single-threaded), so it runs once
CPU_SAMPLES = {"cfg1": (6, 32, 3), "cfg2": (16, 128, 3), "cfg3": (6, 64, 3), "cfg4": (512, 16, 2), "cfg5": (4096, 256, 1)}


def cpu_config(pkg, key, preset, n_prompt, n_dec, max_seq, layout, cpus, want_ids):
    """The reference --stage v2 Model (oracle/_ref) on this host: bench_e2e's once()
    (reset, prefill, n x (sample_greedy + decode)) after one warm-up, median over runs."""
    from oracle.bind import RefModel, ref_available

    if not ref_available():
        return None
    s_prompt, s_dec, runs = CPU_SAMPLES[key]
    s_prompt = min(s_prompt, n_prompt)
    s_dec = min(s_dec, n_dec)
    path, info = ensure_model(pkg, preset, cpus["threads"])
    prompt = pkg.synth_prompt(info["seed"], n_prompt, info["n_vocab"])[:s_prompt]
    ref = RefModel(path, max_seq=max_seq, kv_layout=layout, n_threads=cpus["threads"])
    ref.generate(prompt[: min(len(prompt), 8)], 2)  # warm-up (thread pool, page cache)
    dec, pf, ids = [], [], None
    for _ in range(runs):
        ids, ps, ds = ref.generate(prompt, s_dec)
        dec.append(s_dec / ds)
        pf.append(len(prompt) / ps)
    ref.close()
    full = s_prompt == n_prompt and s_dec == n_dec
    if full:
        sample = f"the full workload ({n_prompt}-token prompt + {n_dec} greedy tokens)"
    elif s_prompt == n_prompt:
        sample = f"the {n_prompt}-token prompt + the first {s_dec} of the {n_dec} greedy tokens"
    else:
        sample = (f"a {s_prompt}-token prefix of the {n_prompt}-token prompt + {s_dec} greedy tokens (the CPU "
                  f"prefill of the whole prompt takes minutes: its attention is single-threaded; decode there "
                  f"reads KV rows of {s_prompt} positions instead of {n_prompt}")
    out = {"value": round(statistics.median(dec), 3), "unit": "tok/s", "cores": cpus["threads"], "kind": "reference",
           "prefill_tok_s": round(statistics.median(pf), 2),
           "sample": f"reference --stage v2 (oracle/_ref, {cpus['threads']} threads): {sample}, median of {runs} "
                     f"run(s) after 1 warm-up"}
    if want_ids is not None and s_prompt == n_prompt:
        out["tokens_match_gpu"] = bool(list(ids) == list(want_ids[: len(ids)]))
    return out


# ---------------------------------------------------------------- main

def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--runs", type=int, default=5, help="bench_e2e runs per config")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--quick", action="store_true", help="headline only (no config list, sweep or prefill leg)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: the token loop runs on one GPU; --gpus {args.gpus} is not supported "
              "(batch-1 decode of a 1.3 GB model fits one MI355X; multi-GPU sharding is design-only)",
              file=sys.stderr)
        return 2
    K, W = args.steps, args.warmup
    _, _, h_preset, h_prompt, _, h_max_seq, h_layout = next(c for c in CONFIGS if c[0] == HEADLINE)
    if K < 1 or h_prompt + max(K, W) > h_max_seq:
        print(f"bench.py: --steps/--warmup must keep {h_prompt} + steps within max-seq {h_max_seq}", file=sys.stderr)
        return 2

    pkg = __graft_entry__.load_package()
    cpus = host_cpus()
    path, info = ensure_model(pkg, h_preset, cpus["threads"])
    prompt = pkg.synth_prompt(info["seed"], h_prompt, info["n_vocab"])

    # ---- headline: W warm-up steps, then K timed steps of the on-device greedy loop
    m = pkg.HipModel(path, max_seq=h_max_seq, kv_layout=h_layout)
    m.prefill(prompt, want_logits=False)
    if W > 0:
        m.generate(W)
    m.reset()
    m.prefill(prompt, want_logits=False)
    t0 = time.perf_counter()
    ids = m.generate(K)  # synchronous: returns after the device finished all K steps
    wall_s = time.perf_counter() - t0
    dev_ms, _, launches, kname = m.last_timing()
    step_bytes = [m.decode_bytes(h_prompt + i) for i in range(K)]
    achieved = sum(step_bytes) / (dev_ms * 1e-3) / 1e9
    dpath = m.decode_path()
    # kernel-by-kernel pass over the same K steps on the graph path (per-class breakdown)
    m.reset()
    m.prefill(prompt, want_logits=False)
    ids_prof, prof = m.profile_generate(K)
    m.close()
    traffic, traffic_src = measured_traffic(HEADLINE, K, kname)
    read_best, read_med, read_cs = pkg.read_stream(4 << 30, iters=10, with_checksum=True)
    copy_best, _ = pkg.copy_stream(COPY_CALIB_BYTES, iters=3)
    value = K / wall_s

    configs = {}
    pf = ctx = None
    if not args.quick:
        for key, desc, preset, n_prompt, n_dec, max_seq, layout in CONFIGS:
            runs = max(1, args.runs if key != "cfg5" else min(args.runs, 3))
            configs[key] = gpu_config(pkg, key, desc, preset, n_prompt, n_dec, max_seq, layout, runs, 2,
                                      cpus["threads"])
            print(f"bench.py: {key} done", file=sys.stderr, flush=True)
        pf = prefill_leg(pkg, cpus["threads"])
        ctx = context_sweep(pkg, cpus["threads"])
    cpu = None
    if not args.no_cpu:
        for key, desc, preset, n_prompt, n_dec, max_seq, layout in CONFIGS:
            if args.quick and key != HEADLINE:
                continue
            want = configs[key]["ids"] if key in configs else list(ids)
            c = cpu_config(pkg, key, preset, n_prompt, n_dec, max_seq, layout, cpus, want)
            if key in configs:
                configs[key]["cpu_baseline"] = c
            if key == HEADLINE:
                cpu = c
            print(f"bench.py: {key} cpu baseline done", file=sys.stderr, flush=True)
        if pf is not None and configs.get("cfg4", {}).get("cpu_baseline"):
            pf["cpu_baseline_prefill_tok_s"] = configs["cfg4"]["cpu_baseline"]["prefill_tok_s"]
    for c in configs.values():
        c.pop("ids", None)

    out = {
        "metric": "decode tok/s & % of HBM roofline, Llama-3.2-1B-shape Q8_0, batch 1",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall_s * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / PUBLISHED_CPU_TOK_S, 1),
        "vs_baseline_ref": f"{PUBLISHED_CPU_TOK_S} tok/s: reference --stage v2, Llama-3.2-1B Q8_0, "
                           "Ryzen 5 4600H 6c/12t (published)",
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Llama-3.2-1B-shape Q8_0 synthetic GGUF (L16 D2048 H32/8 hd64 F8192 V128256, tied "
                        "lm_head, N(0,0.02) seed 42), 6-token prompt, greedy decode, max-seq 512, batch 1",
            "prompt_tokens": h_prompt,
            "decode_tokens": K,
            "max_seq": h_max_seq,
            "weights": "Q8_0",
            "kv_cache": "fp32 seq-major",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": kname,
            "launches": launches,
            "bytes_per_launch": round(sum(step_bytes) / launches),
            "avg_launch_us": round(dev_ms / launches * 1e3, 3),
        },
        "cpu_baseline": cpu,
        "host_cpus": cpus,
        "step_hbm_gb_s": round(sum(step_bytes) / wall_s / 1e9, 1),
        "read_stream_gb_s": round(read_best, 1),
        "read_stream_median_gb_s": round(read_med, 1),
        "read_stream_checksum_ok": read_cs == pkg.stream_checksum(4 << 30),
        "copy_stream_gb_s": round(copy_best, 1),
        "frac_of_read_stream": round(achieved / read_best, 4),
        "bytes_per_step": round(statistics.mean(step_bytes)),
        "device_ms_per_step": round(dev_ms / K, 4),
        "decode_path": "persistent step kernel" if dpath == 1 else "graph",
        "graph_kernel_ms_by_class": {k: round(v[0] / K, 4) for k, v in prof.items()},
        "tokens_match_profile_pass": bool(list(ids) == list(ids_prof)),
        "configs": configs,
        "prefill": pf,
        "context_sweep": ctx,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
