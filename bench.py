"""Decode throughput of tinferno's token loop on one MI355X.

Workload: the Llama-3.2-1B-shape Q8_0 synthetic GGUF (16 layers, d_model 2048, 32/8 heads,
head_dim 64, FFN 8192, vocab 128256, tied lm_head, seed 42), a 6-token prompt from the
seed, greedy decode at batch 1, max-seq 512. A step is one decode token: embedding, 16
layers, final norm, lm_head and the greedy argmax (Model::decode + sample_greedy).

    python bench.py [--gpus 1] [--steps 32] [--warmup 8] [--no-cpu]

Prints one JSON line. `value` is decode tok/s of K steps of the on-device greedy loop
(tf_hip_generate: one persistent step-kernel launch for the K steps, inputs resident in
HBM), timed between two synchronisations. `roofline` is that kernel's achieved
algorithmic GB/s (the K steps' bytes over the HIP-event time of the launch); a second,
kernel-by-kernel pass over the same steps on the graph path gives the per-class times;
`cpu_baseline` is the reference --stage v2 path (compiled from its own sources) timed
on this host's cores over the same prompt and steps. `prefill` is the 512-token prompt
workload of the same model on the matrix cores: tok/s from HIP events around the call,
algorithmic TFLOP/s and their fraction of the dense fp16 MFMA peak, the decode rate
after the prompt, and the reference CPU prefill on a bounded sample. `context_sweep` is the
decode rate after prompts of 512..4000 tokens in a 4096-position cache (graph path).
`other_configs` runs the other workloads at their own shapes (Qwen2.5-0.5B with QKV bias,
the mixed Q4 file, Qwen2.5-1.5B after a 4096-token prompt): prefill and decode tok/s and
decode GB/s.
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

PRESET = "llama1b_q8"
PROMPT_TOKENS = 6
MAX_SEQ = 512
HBM_PEAK_GBS = 8000.0
COPY_CALIB_BYTES = 1 << 30
TRAFFIC_SUMMARY = ROOT / "profiles" / "decode_llama1b_q8_0_traffic.txt"
STEP_TRAFFIC_SUMMARY = ROOT / "profiles" / "decode_llama1b_q8_0_step_kernel_traffic.txt"
PUBLISHED_CPU_TOK_S = 10.74  # reference --stage v2, Llama-3.2-1B Q8_0, Ryzen 5 4600H 6c/12t (its published figure)
# prefill leg: a 512-token prompt of the same model, then 16 decode tokens
PF_PROMPT_TOKENS = 512
PF_DECODE_TOKENS = 16
PF_MAX_SEQ = 1024
PF_REPS = 5
PF_CPU_SAMPLE_TOKENS = 64
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X
# context sweep: decode after prompts of these lengths, cache of CTX_MAX_SEQ positions
CTX_PROMPTS = (512, 1024, 2048, 4000)
CTX_MAX_SEQ = 4096
CTX_STEPS = 16


def host_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def model_path() -> str:
    d = pathlib.Path(tempfile.gettempdir()) / "tinferno_bench"
    d.mkdir(parents=True, exist_ok=True)
    return str(d / f"{PRESET}-seed42.gguf")


def measured_traffic(kernel_class: str, tokens_per_launch: int = 1):
    """HBM bytes per launch of `kernel_class` from the committed counter summaries (two
    rocprofv3 --pmc runs, FETCH_SIZE then WRITE_SIZE, scaled by the counters of a
    known-size copy); the step kernel's summary is per decoded token. None when no
    summary covers it."""
    for path, key, mult in ((TRAFFIC_SUMMARY, "traffic_bytes_per_launch", 1),
                            (STEP_TRAFFIC_SUMMARY, "traffic_bytes_per_token", tokens_per_launch)):
        try:
            for line in path.read_text().splitlines():
                f = line.split()
                if len(f) == 3 and f[0] == key and f[1] == kernel_class:
                    return int(float(f[2]) * mult)
        except OSError:
            pass
    return None


def prefill_flops(info, n):
    """Algorithmic FLOP of a prefill of n tokens: 2 per weight per token for the layer
    matrices, the causal attention (q.k and p.v over i + 1 positions for token i), and
    the lm_head of the last token."""
    D, F, L, H, G = info["n_embd"], info["n_ff"], info["n_layer"], info["n_head"], info["n_kv_head"]
    hd = D // H
    dense = 2.0 * n * L * (D * (H * hd + 2 * G * hd) + H * hd * D + 3 * D * F)
    attn = 4.0 * hd * (n * (n + 1) / 2) * H * L
    return dense + attn + 2.0 * D * info["n_vocab"], dense


def prefill_leg(pkg, path, info):
    """The 512-token prompt: PF_REPS timed prefills from a reset (device ms from HIP events
    around the call's kernels, and wall ms of the synchronous call), then the 16 decode
    tokens after it."""
    prompt = pkg.synth_prompt(info["seed"], PF_PROMPT_TOKENS, info["n_vocab"])
    m = pkg.HipModel(path, max_seq=PF_MAX_SEQ, kv_layout=0)
    m.prefill(prompt, want_logits=False)  # warm-up
    dev, wall = [], []
    for _ in range(PF_REPS):
        m.reset()
        t0 = time.perf_counter()
        _, am = m.prefill(prompt, want_logits=False)
        wall.append((time.perf_counter() - t0) * 1e3)
        ms, _, _, name = m.last_timing()
        dev.append(ms)
    ids = m.generate(PF_DECODE_TOKENS)
    dec_ms = m.last_timing()[0]
    pf_path = m.prefill_path()
    m.close()
    flops, dense = prefill_flops(info, PF_PROMPT_TOKENS)
    d_ms = statistics.median(dev)
    tflops = flops / (d_ms * 1e-3) / 1e12
    return {
        "workload": f"{PF_PROMPT_TOKENS}-token prompt (uniform ids, seed {info['seed']}) of the same model, "
                    f"max-seq {PF_MAX_SEQ}, then {PF_DECODE_TOKENS} greedy decode tokens",
        "path": name if pf_path == m.PREFILL_MFMA else "per-token",
        "tokens": PF_PROMPT_TOKENS,
        "device_ms": round(d_ms, 3),
        "wall_ms": round(statistics.median(wall), 3),
        "tok_s": round(PF_PROMPT_TOKENS / (d_ms * 1e-3), 1),
        "tflop": round(flops / 1e12, 4),
        "dense_tflop": round(dense / 1e12, 4),
        "achieved_tflop_s": round(tflops, 2),
        "mfma_peak_tflop_s": MFMA_F16_PEAK_TFLOPS,
        "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "mfma_note": "algorithmic FLOP/s over the dense fp16 MFMA peak; the GEMMs issue two fp16 MFMAs "
                     "(activation hi and lo) per algorithmic product, attention runs on fp32 MFMA",
        "first_token": int(am),
        "decode_after_prompt_tok_s": round(PF_DECODE_TOKENS / (dec_ms * 1e-3), 1),
    }


def context_sweep(pkg, path, info):
    """Decode rate by context length (the sweep the reference's roofline.py reads as
    bench "context" and its runs never produced): per prompt length, a prefill from a
    reset, then CTX_STEPS greedy tokens timed by HIP events; GB/s counts the weights once
    and the KV rows of every position read (tf_hip_decode_bytes)."""
    m = pkg.HipModel(path, max_seq=CTX_MAX_SEQ, kv_layout=0)
    # warm-up: the step kernel's one-time set-up and first launches stay out of the points
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


# the other configurations of the workload list: (name, preset, prompt tokens, decode tokens,
# max-seq, KV layout)
OTHER_CONFIGS = (
    ("qwen2.5-0.5b-shape q8_0 + qkv bias", "qwen05b_q8", 16, 128, 512, 0),
    ("llama-3.2-1b-shape mixed q4_0/q4_1/q6_k", "llama1b_mixq4", 6, 64, 512, 0),
    ("qwen2.5-1.5b-shape q8_0, 4096-token prompt, head-major cache", "qwen15b_q8", 4096, 256, 8192, 1),
)


def configs_leg(pkg):
    """The other workloads at their own shapes: a prefill of the prompt from a reset, then
    the decode tokens in one greedy generate call (both timed by the HIP events around
    the call's kernels); GB/s counts each step's weights once and its KV rows
    (tf_hip_decode_bytes), as for the headline."""
    out = []
    for name, preset, n_prompt, n_dec, max_seq, layout in OTHER_CONFIGS:
        info = pkg.synth_preset_info(preset)
        path = str(pathlib.Path(model_path()).parent / f"{preset}-seed{info['seed']}.gguf")
        if not os.path.exists(path):
            pkg.synth_write(preset, path, threads=host_threads())
        prompt = pkg.synth_prompt(info["seed"], n_prompt, info["n_vocab"])
        m = pkg.HipModel(path, max_seq=max_seq, kv_layout=layout)
        m.prefill(prompt, want_logits=False)  # warm-up (and one-time weight packing)
        m.generate(8)
        m.reset()
        m.prefill(prompt, want_logits=False)
        pf_ms, _, _, pf_name = m.last_timing()
        m.generate(n_dec)
        ms, _, _, dec_name = m.last_timing()
        b = sum(m.decode_bytes(n_prompt + i) for i in range(n_dec))
        gbs = b / (ms * 1e-3) / 1e9
        out.append({"workload": name, "prompt_tokens": n_prompt, "decode_tokens": n_dec, "max_seq": max_seq,
                    "prefill_tok_s": round(n_prompt / (pf_ms * 1e-3), 1), "prefill_path": pf_name,
                    "decode_tok_s": round(n_dec / (ms * 1e-3), 1), "decode_gb_s": round(gbs, 1),
                    "decode_hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "decode_path": dec_name,
                    "bytes_per_step": round(b / n_dec)})
        m.close()
    return out


def cpu_prefill_baseline(pkg, path, info):
    """The reference --stage v2 prefill (oracle/_ref) on this host's cores over the first
    PF_CPU_SAMPLE_TOKENS tokens of the 512-token prompt (a bounded sample: its cost per
    token is the dense layers', as at 512 tokens): median of 3 runs after a warm-up."""
    from oracle.bind import RefModel, ref_available

    if not ref_available():
        return None
    threads = host_threads()
    prompt = pkg.synth_prompt(info["seed"], PF_PROMPT_TOKENS, info["n_vocab"])[:PF_CPU_SAMPLE_TOKENS]
    ref = RefModel(path, max_seq=PF_MAX_SEQ, kv_layout=0, n_threads=threads)
    runs = []
    for i in range(4):
        ref.reset()
        t0 = time.perf_counter()
        ref.prefill(prompt)
        if i:
            runs.append(len(prompt) / (time.perf_counter() - t0))
    ref.close()
    return {
        "value": round(statistics.median(runs), 2),
        "unit": "tok/s",
        "cores": threads,
        "kind": "reference",
        "sample": f"reference --stage v2 prefill (oracle/_ref, {threads} threads) of the first "
                  f"{PF_CPU_SAMPLE_TOKENS} tokens of the {PF_PROMPT_TOKENS}-token prompt, median of 3 runs "
                  "after 1 warm-up",
    }


def cpu_baseline(path, prompt, n_decode, want_ids):
    """The reference --stage v2 Model (oracle/_ref) on this host: bench_e2e's once()
    (reset, prefill, n x (sample_greedy + decode)), 1 warm-up + 3 runs, median tok/s."""
    from oracle.bind import RefModel, ref_available

    if not ref_available():
        return None, None
    threads = host_threads()
    ref = RefModel(path, max_seq=MAX_SEQ, kv_layout=0, n_threads=threads)
    ref.generate(prompt, min(4, n_decode))
    runs = []
    ids = None
    for _ in range(3):
        ids, _, dec_s = ref.generate(prompt, n_decode)
        runs.append(n_decode / dec_s)
    ref.close()
    base = {
        "value": round(statistics.median(runs), 3),
        "unit": "tok/s",
        "cores": threads,
        "kind": "reference",
        "sample": f"reference --stage v2 (oracle/_ref, {threads} threads): {PROMPT_TOKENS}-token prompt + "
                  f"{n_decode} greedy decode tokens of the same model, median of 3 runs after 1 warm-up",
    }
    match = bool(want_ids is not None and list(ids) == list(want_ids[: len(ids)]))
    return base, match


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: the token loop runs on one GPU; --gpus {args.gpus} is not supported "
              "(batch-1 decode of a 1.3 GB model fits one MI355X; multi-GPU sharding is design-only)",
              file=sys.stderr)
        return 2
    K, W = args.steps, args.warmup
    if K < 1 or PROMPT_TOKENS + max(K, W) > MAX_SEQ:
        print(f"bench.py: --steps/--warmup must keep {PROMPT_TOKENS} + steps within max-seq {MAX_SEQ}",
              file=sys.stderr)
        return 2

    pkg = __graft_entry__.load_package()
    path = model_path()
    info = pkg.synth_preset_info(PRESET)
    if not os.path.exists(path):
        t0 = time.time()
        pkg.synth_write(PRESET, path, threads=host_threads())
        print(f"bench.py: wrote {path} in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    prompt = pkg.synth_prompt(info["seed"], PROMPT_TOKENS, info["n_vocab"])

    m = pkg.HipModel(path, max_seq=MAX_SEQ, kv_layout=0)
    # warm-up: W untimed decode steps
    m.prefill(prompt, want_logits=False)
    if W > 0:
        m.generate(W)
    # timed: K greedy decode steps after an untimed prefill
    m.reset()
    t0 = time.perf_counter()
    m.prefill(prompt, want_logits=False)
    prefill_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    ids = m.generate(K)  # synchronous: returns after the device finished all K steps
    wall_s = time.perf_counter() - t0
    dev_ms, _, _, _ = m.last_timing()
    ms_per_step = wall_s * 1e3 / K
    value = K / wall_s
    # algorithmic bytes of the K steps (weights once per step, one embedding row, the KV cache)
    step_bytes = [m.decode_bytes(PROMPT_TOKENS + i) for i in range(K)]
    step_gbs = sum(step_bytes) / wall_s / 1e9

    dpath = m.decode_path()
    # kernel-by-kernel pass over the same K steps on the graph path (per-class breakdown)
    m.reset()
    m.prefill(prompt, want_logits=False)
    ids_prof, prof = m.profile_generate(K)
    if dpath == m.PATH_STEP:
        # the decode kernel is the one persistent launch of the timed generate(K): its
        # algorithmic bytes are the K steps', its duration the HIP events around it
        dom, d_launch, d_bytes, d_ms = "k_step", 1, float(sum(step_bytes)), dev_ms
    else:
        dom = max(prof, key=lambda k: prof[k][0])
        d_ms, d_launch, d_bytes = prof[dom]
    achieved = (d_bytes / d_launch) / (d_ms / d_launch * 1e-3) / 1e9
    m.close()
    read_best, read_med = pkg.read_stream(4 << 30, iters=10)
    # known-size copy: the reference dispatch for the HBM byte counters (FETCH_SIZE, WRITE_SIZE)
    copy_best, _ = pkg.copy_stream(COPY_CALIB_BYTES, iters=3)

    pf = prefill_leg(pkg, path, info)
    ctx = context_sweep(pkg, path, info)
    others = configs_leg(pkg)
    cpu, match = (None, None) if args.no_cpu else cpu_baseline(path, prompt, K, ids)
    if not args.no_cpu:
        pf["cpu_baseline"] = cpu_prefill_baseline(pkg, path, info)

    out = {
        "metric": "decode tok/s & % of HBM roofline, Llama-3.2-1B-shape Q8_0, batch 1",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
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
            "prompt_tokens": PROMPT_TOKENS,
            "decode_tokens": K,
            "max_seq": MAX_SEQ,
            "weights": "Q8_0",
            "kv_cache": "fp32 seq-major",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(dom, K if dom == "k_step" else 1),
            "kernel": dom,
            "launches": d_launch,
            "bytes_per_launch": round(d_bytes / d_launch),
            "avg_launch_us": round(d_ms / d_launch * 1e3, 3),
        },
        "step_hbm_gb_s": round(step_gbs, 1),
        "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "read_stream_gb_s": round(read_best, 1),
        "copy_stream_gb_s": round(copy_best, 1),
        "step_frac_of_read_stream": round(step_gbs / read_best, 4),
        "bytes_per_step": round(statistics.mean(step_bytes)),
        "device_ms_per_step": round(dev_ms / K, 4),
        "prefill_6_tokens_wall_ms": round(prefill_s * 1e3, 3),
        "prefill": pf,
        "context_sweep": ctx,
        "other_configs": others,
        "decode_path": "persistent step kernel" if dpath == 1 else "graph",
        "graph_kernel_ms_by_class": {k: round(v[0] / K, 4) for k, v in prof.items()},
        "tokens_match_profile_pass": bool(list(ids) == list(ids_prof)),
        "tokens_match_reference": match,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
