"""Summaries of rocprofv3 CSV output for the decode step, as short text.

    python3 agent-serve_amd/profsum.py trace <kernel_stats.csv> [--steps K]
    python3 agent-serve_amd/profsum.py steps <kernel_trace.csv>
    python3 agent-serve_amd/profsum.py stepcounters <fetch counter_collection.csv> <write counter_collection.csv>
        --copy-fetch <csv> --copy-write <csv> [--copy-bytes N] [--kernel <name>]
    python3 agent-serve_amd/profsum.py digest
    python3 agent-serve_amd/profsum.py decodetrace <kernel_stats.csv> <kernel_trace.csv> [--kernel <name>]
        [--algo-bytes B]
    python3 agent-serve_amd/profsum.py traffic <fetch counter_collection.csv> <write counter_collection.csv>
        --copy-bytes N [--copy-fetch <csv> --copy-write <csv>]
    python3 agent-serve_amd/profsum.py prefill <kernel_trace.csv> --tokens N --dims D,F,L,H,G

`trace` lists each kernel's calls and average / min duration from a --kernel-trace --stats
run. `traffic` turns the FETCH_SIZE and WRITE_SIZE counters (KiB per dispatch, one
--pmc run each) into HBM bytes per dispatch, each scaled by what the same counter reads
for k_copy_stream, which reads N bytes and writes N bytes; the last line,
`traffic_bytes_per_launch <kernel> <bytes>`, is what bench.py reads back. `stepcounters`
does the same for the persistent decode kernel (`traffic_bytes_per_token <kernel> <bytes>`)
with the scale factors of a separate k_copy_stream run, and ends with the provenance lines
bench.py checks: `commit <sha>` and `csrc_sha256 <digest of the kernel sources>`.
"""
from __future__ import annotations

import argparse
import collections
import csv
import hashlib
import pathlib
import re
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]


def kernel_source_digest() -> str:
    """sha256 (first 16 hex digits) of the kernel sources (agent-serve_amd/csrc/*) and the
    ABI header: a counter summary records the digest of the build it measured, and bench.py
    uses a summary's figures only while the digest is that of the sources it runs."""
    h = hashlib.sha256()
    files = sorted((ROOT / "agent-serve_amd" / "csrc").glob("*")) + [ROOT / "include" / "tf_hip.h"]
    for f in files:
        if f.is_file():
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:16]


def provenance(commit: str | None) -> None:
    """The lines bench.py reads back: the commit measured and the kernel-source digest."""
    if not commit:
        try:
            commit = subprocess.run(["git", "-C", str(ROOT), "rev-parse", "--short=12", "HEAD"], capture_output=True,
                                    text=True, check=True).stdout.strip()
        except (OSError, subprocess.CalledProcessError):
            commit = "unknown"
    print(f"commit {commit}")
    print(f"csrc_sha256 {kernel_source_digest()}")


def short(name: str) -> str:
    name = re.sub(r"\(tfk::[A-Za-z]+\)$", "", name)
    name = name.replace("tfk::gemv_detail::", "").replace("tfk::(anonymous namespace)::", "")
    return re.sub(r"^void ", "", name)[:60]


def decode_class(name: str) -> str:
    """Kernel class of a decode-step dispatch, as tf_hip_profile_generate names them: the
    GEMV's epilogue mode (0 store, 1 residual, 2 SiLU*up, 3 logits) and steps per tile U
    tell the QKV, wo, gate/up, down and lm_head launches apart."""
    m = re.search(r"k_gemv<(\d+), (\d+), (\d+), (\d+)>", name)
    if m:
        mode, u = int(m.group(3)), int(m.group(4))
        return {0: "qkv_gemv", 2: "gateup_gemv", 3: "lmhead_gemv"}.get(mode, "down_gemv" if u == 4 else "wo_gemv")
    for key, cls in (("k_attn_decode", "attention"), ("k_attn_combine", "attention"), ("k_embed", "embed"),
                     ("k_step", "k_step")):
        if key in name:
            return cls
    return short(name).replace(" ", "")


def step_dispatches(trace_csv: str) -> list[float]:
    """Durations (us) of each k_step dispatch, in launch order."""
    out = []
    for r in csv.DictReader(open(trace_csv)):
        if "k_step" in r["Kernel_Name"]:
            out.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return out


def copy_scales(fetch_csv: str, write_csv: str, copy_bytes: int) -> tuple[float, float]:
    """FETCH_SIZE and WRITE_SIZE scale factors: bytes over the counter's KiB for
    k_copy_stream, which reads copy_bytes and writes copy_bytes per dispatch."""
    f = counter_means(fetch_csv, "FETCH_SIZE")
    w = counter_means(write_csv, "WRITE_SIZE")
    fk = next(k for k in f if "k_copy_stream" in k)
    wk = next(k for k in w if "k_copy_stream" in k)
    return copy_bytes / (f[fk][1] * 1024.0), copy_bytes / (w[wk][1] * 1024.0)


def step_counters(fetch_csv: str, write_csv: str, f_scale: float, w_scale: float, kernel: str = "k_step") -> None:
    """HBM bytes per decode token of the persistent decode kernel (k_step) from a
    run of the CLI (the prompt, then one launch per decoded token): the median over the
    launches after the first, FETCH_SIZE and WRITE_SIZE scaled by the copy kernel's
    factors."""
    def vals(p, c):
        return [float(r["Counter_Value"]) for r in csv.DictReader(open(p))
                if r["Counter_Name"] == c and kernel in r["Kernel_Name"]]
    f, w = vals(fetch_csv, "FETCH_SIZE"), vals(write_csv, "WRITE_SIZE")
    fm, wm = sorted(f[1:])[len(f[1:]) // 2], sorted(w[1:])[len(w[1:]) // 2]
    print(f"{kernel} dispatches: {len(f)} (one per decoded token; the first, a cold start, is left out of the medians)")
    print(f"decode dispatches: FETCH_SIZE median {fm:.0f} KiB (min {min(f[1:]):.0f}, max {max(f[1:]):.0f}), "
          f"WRITE_SIZE median {wm:.0f} KiB (min {min(w[1:]):.0f}, max {max(w[1:]):.0f})")
    print(f"scale factors (k_copy_stream): FETCH_SIZE x {f_scale:.4f}, WRITE_SIZE x {w_scale:.4f}")
    print(f"traffic_bytes_per_token {kernel} {fm * 1024 * f_scale + wm * 1024 * w_scale:.0f}")


def pf_classifier():
    """Kernel name -> prefill class, for dispatches in launch order (the attn_output and
    ffn_down GEMMs share a kernel and alternate); None for kernels outside the prefill."""
    resid = [0]

    def classify(k: str):
        if "k_pf_" not in k and "k_embed_rows" not in k:
            return None
        if "k_pf_reduce" in k:
            return "splitk_reduce"
        if re.search(r"k_pf_gemm_(q8|big|split)<0", k):
            return "qkv_gemm"
        if re.search(r"k_pf_gemm_(q8|big|split)<1", k):
            resid[0] += 1
            return "wo_gemm" if resid[0] % 2 == 1 else "down_gemm"
        if re.search(r"k_pf_gemm_(q8|big|split)<2", k):
            return "gateup_gemm"
        if "k_pf_attn" in k:
            return "attention"
        return re.sub(r"^_ZN3tfk12_GLOBAL__N_1\d+", "", short(k)).split("(")[0].split("E")[0]

    return classify


def mfma(counter_csv: str, simds: int, xcds: int) -> None:
    """Matrix-core work per prefill class from one --pmc pass with SQ_INSTS_VALU_MFMA_MOPS_F16,
    SQ_INSTS_VALU_MFMA_MOPS_F32, SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE: MFMA FLOP
    (MOPS x 512) per call and the share of SIMD cycles the matrix cores were busy
    (busy cycles / (one XCD's active cycles x SIMDs), as rocprofv3's MfmaUtil)."""
    rows = collections.defaultdict(dict)  # dispatch id -> counter -> value
    names = {}
    for r in csv.DictReader(open(counter_csv)):
        d, c, v = int(r["Dispatch_Id"]), r["Counter_Name"], float(r["Counter_Value"])
        rows[d][c] = rows[d].get(c, 0.0) + v
        names[d] = r["Kernel_Name"]
    classify = pf_classifier()
    acc = collections.defaultdict(lambda: [0, 0.0, 0.0, 0.0, 0.0])
    for d in sorted(rows):
        c = classify(names[d])
        if c is None:
            continue
        v = rows[d]
        a = acc[c]
        a[0] += 1
        a[1] += v.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) * 512
        a[2] += v.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0) * 512
        a[3] += v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        # GRBM_GUI_ACTIVE comes summed over the XCDs: one XCD's active cycles are value / xcds
        a[4] += v.get("GRBM_GUI_ACTIVE", 0.0) / xcds * simds
    print(f"{'class':16s} {'calls':>6s} {'F16 GFLOP/call':>15s} {'F32 GFLOP/call':>15s} {'MFMA busy':>10s}")
    for c, (n, f16, f32, busy, active) in sorted(acc.items(), key=lambda kv: -kv[1][3]):
        print(f"{c:16s} {n:6d} {f16 / n / 1e9:15.2f} {f32 / n / 1e9:15.2f} {busy / max(active, 1):10.1%}")


def prefill(trace_csv: str, n: int, dims: str) -> None:
    """Per kernel class of one prompt prefill (the k_pf_* dispatches of the trace): launches,
    average and total microseconds, algorithmic FLOP per launch and TFLOP/s. Dense GEMM
    FLOP are 2 per weight per row; attention's are q.k and p.v over i + 1 positions for
    row i. FLOP and TFLOP/s come from the prompt's total per class over the class's total
    time, so a prompt run in several chunks (one launch per chunk and layer) counts right.
    The attn_output and ffn_down GEMMs share a kernel and alternate in launch order."""
    D, F, L, H, G = (int(v) for v in dims.split(","))
    hd = D // H
    flop = {  # per layer, the whole prompt
        "qkv_gemm": 2.0 * n * D * (H * hd + 2 * G * hd),
        "wo_gemm": 2.0 * n * H * hd * D,
        "gateup_gemm": 2.0 * n * D * 2 * F,
        "down_gemm": 2.0 * n * F * D,
        "attention": 4.0 * hd * (n * (n + 1) / 2) * H,
    }
    acc: dict[str, list[float]] = collections.defaultdict(list)
    classify = pf_classifier()
    for r in csv.DictReader(open(trace_csv)):
        c = classify(r["Kernel_Name"])
        if c is None:
            continue
        acc[c].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in acc.values())
    print(f"prefill of {n} tokens, {L} layers: {total / 1e3:.3f} ms in k_pf_* kernels")
    print(f"{'class':16s} {'calls':>6s} {'avg_us':>9s} {'total_ms':>9s} {'share':>6s} {'GFLOP/call':>11s} {'TFLOP/s':>8s}")
    for c, v in sorted(acc.items(), key=lambda kv: -sum(kv[1])):
        avg = sum(v) / len(v)
        f = flop.get(c)
        fs = (f"{f * L / len(v) / 1e9:11.2f} {f * L / (sum(v) * 1e-6) / 1e12:8.1f}" if f else f"{'':11s} {'':8s}")
        print(f"{c:16s} {len(v):6d} {avg:9.2f} {sum(v) / 1e3:9.3f} {sum(v) / total:6.1%} {fs}")


def trace(path: str, steps: int | None) -> None:
    rows = list(csv.DictReader(open(path)))
    print(f"{'kernel':60s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'total_ms':>9s}")
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        print(f"{short(r['Name']):60s} {int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.2f} "
              f"{float(r['MinNs']) / 1e3:9.2f} {float(r['TotalDurationNs']) / 1e6:9.3f}")


def decode_trace(stats_csv: str, trace_csv: str, kernel: str, algo_bytes: float | None) -> None:
    """A decode run of the CLI (one launch of the persistent kernel per decoded token): the
    kernel table, every dispatch of `kernel` in launch order, their median after the first
    (a cold start) and, given the algorithmic bytes per token, the rate and its share of
    8 TB/s."""
    trace(stats_csv, None)
    d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in csv.DictReader(open(trace_csv))
         if kernel in r["Kernel_Name"]]
    print()
    print(f"Per {kernel} dispatch (us), in launch order (one decoded token each):")
    for i in range(0, len(d), 16):
        print(" ".join(f"{v:.1f}" for v in d[i:i + 16]))
    rest = sorted(d[1:])
    med = rest[len(rest) // 2]
    line = f"{kernel} dispatches after the first: median {med:.1f} us ({rest[0]:.1f}-{rest[-1]:.1f})"
    if algo_bytes:
        tbs = algo_bytes / (med * 1e-6) / 1e12
        line += f"; algorithmic bytes per token {algo_bytes:,.0f}: {tbs:.2f} TB/s, {tbs / 8.0:.1%} of 8 TB/s"
    print(line + ".")
    print(f"median_us {kernel} {med:.1f}")


def counter_means(path: str, counter: str) -> dict[str, tuple[int, float]]:
    """Mean counter value per kernel name; for k_step (one launch per call, calls of
    different token counts) the largest dispatch, which is the longest generate call."""
    acc: dict[str, list[float]] = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter:
            acc[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return {k: (len(v), max(v) if "k_step" in k else sum(v) / len(v)) for k, v in acc.items()}


def traffic(fetch_csv: str, write_csv: str, copy_bytes: int, scales: tuple[float, float] | None = None) -> None:
    """Per kernel: HBM bytes per dispatch. The scale factors come from k_copy_stream in the
    same files, or from a separate calibration run (scales)."""
    fetch = counter_means(fetch_csv, "FETCH_SIZE")
    write = counter_means(write_csv, "WRITE_SIZE")
    copy_key = next((k for k in fetch if "k_copy_stream" in k), None)
    if scales:
        f_scale, w_scale = scales
        print(f"scale factors (k_copy_stream of {copy_bytes} bytes, separate run): fetch {f_scale:.4f}, write {w_scale:.4f}")
    else:
        f_scale = copy_bytes / (fetch[copy_key][1] * 1024.0)
        w_scale = copy_bytes / (write[copy_key][1] * 1024.0)
        print(f"k_copy_stream of {copy_bytes} bytes: FETCH_SIZE {fetch[copy_key][1]:.0f} KiB, "
              f"WRITE_SIZE {write[copy_key][1]:.0f} KiB -> scale fetch {f_scale:.4f}, write {w_scale:.4f}")
    print(f"{'kernel':60s} {'n':>5s} {'fetch_KiB':>11s} {'write_KiB':>10s} {'hbm_bytes':>12s}")
    for k, (n, f) in sorted(fetch.items(), key=lambda kv: -kv[1][1]):
        if k == copy_key:
            continue
        w = write.get(k, (0, 0.0))[1]
        b = f * 1024.0 * f_scale + w * 1024.0 * w_scale
        print(f"{short(k):60s} {n:5d} {f:11.1f} {w:10.1f} {b:12.0f}")
    for k, (n, f) in fetch.items():
        if k == copy_key:
            continue
        w = write.get(k, (0, 0.0))[1]
        print(f"traffic_bytes_per_launch {decode_class(k)} {f * 1024.0 * f_scale + w * 1024.0 * w_scale:.0f}")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("what", choices=["trace", "traffic", "steps", "stepcounters", "prefill", "mfma", "digest",
                                     "decodetrace"])
    ap.add_argument("--algo-bytes", type=float, default=None, help="decodetrace: algorithmic bytes per token")
    ap.add_argument("files", nargs="*")
    ap.add_argument("--copy-fetch", help="FETCH_SIZE counter csv of the k_copy_stream calibration run")
    ap.add_argument("--copy-write", help="WRITE_SIZE counter csv of the k_copy_stream calibration run")
    ap.add_argument("--kernel", default="k_step", help="stepcounters, decodetrace: the persistent decode kernel's name")
    ap.add_argument("--commit", default=None, help="commit measured (default: git HEAD)")
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--copy-bytes", type=int, default=1 << 30)
    ap.add_argument("--tokens", type=int, default=512)
    ap.add_argument("--dims", default="2048,8192,16,32,8", help="D,F,L,H,G")
    ap.add_argument("--simds", type=int, default=1024, help="SIMDs of the GPU (MI355X: 256 CUs x 4)")
    ap.add_argument("--xcds", type=int, default=8, help="XCDs of the GPU (MI355X: 8)")
    a = ap.parse_args()
    if a.what == "trace":
        trace(a.files[0], a.steps)
        provenance(a.commit)
    elif a.what == "decodetrace":
        decode_trace(a.files[0], a.files[1], a.kernel, a.algo_bytes)
        provenance(a.commit)
    elif a.what == "prefill":
        prefill(a.files[0], a.tokens, a.dims)
        provenance(a.commit)
    elif a.what == "mfma":
        mfma(a.files[0], a.simds, a.xcds)
        provenance(a.commit)
    elif a.what == "stepcounters":
        fs, ws = copy_scales(a.copy_fetch, a.copy_write, a.copy_bytes)
        step_counters(a.files[0], a.files[1], fs, ws, a.kernel)
        provenance(a.commit)
    elif a.what == "digest":
        provenance(a.commit)
    elif a.what == "steps":
        for i, d in enumerate(step_dispatches(a.files[0])):
            print(f"k_step dispatch {i}: {d:9.1f} us")
    else:
        scales = copy_scales(a.copy_fetch, a.copy_write, a.copy_bytes) if a.copy_fetch and a.copy_write else None
        traffic(a.files[0], a.files[1], a.copy_bytes, scales)
        provenance(a.commit)
    return 0


if __name__ == "__main__":
    sys.exit(main())
