"""Writes the long-context fixture from the reference: the Qwen2.5-1.5B-shape Q8_0 model
after a 4096-token prompt.

Workload: the qwen15b_q8 synthetic GGUF (28 layers, d_model 1536, 12/2 heads, head_dim 128,
FFN 8960, vocab 151936, QKV bias, tied, seed 42), a 4096-token prompt drawn from the seed,
head-major fp32 KV cache, max-seq 8192, then 256 greedy decode tokens.

1. The reference compiled from its own sources (oracle/_ref/libref.so, --stage v2 Model)
   runs the workload: greedy ids, and per step (after the prefill and after each decode)
   the top-8 logits and the sha256 of the whole fp32 logits vector.
2. The oracle runs the same workload; its logits must equal the reference's bit for bit at
   every step. The reference exposes no per-layer activations, so the last step's taps
   (residual after layers 0, 7, 14, 21 and 27, and the output-normed vector) come from the
   oracle run, which the step hashes tie to the reference.

Takes several minutes of CPU (the reference's prompt attention is single-threaded).

    python tests/golden/make_golden_long.py [--threads N]
"""
from __future__ import annotations

import argparse
import hashlib
import pathlib
import sys
import tempfile
import time

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402
from oracle.bind import OracleModel, RefModel  # noqa: E402

PRESET = "qwen15b_q8"
N_PROMPT = 4096
N_GEN = 256
MAX_SEQ = 8192
LAYOUT = 1  # head-major
TOPK = 8
TAP_LAYERS = (0, 7, 14, 21, 27, 28)  # 28 = the output-normed vector fed to the lm_head
OUT = HERE / "qwen15b_4096.npz"


def file_sha(path: str) -> bytes:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.digest()


def run(model, prompt, log):
    """prefill, then N_GEN x (argmax, decode): ids, per-step top-k and logits digests."""
    t0 = time.time()
    logits = model.prefill(prompt)
    log(f"prefill {len(prompt)} tokens: {time.time() - t0:.1f}s")
    ids, top_i, top_v, shas = [], [], [], []

    def record(lg):
        order = np.argsort(-lg, kind="stable")[:TOPK]
        top_i.append(order.astype(np.int32))
        top_v.append(lg[order].astype(np.float32))
        shas.append(np.frombuffer(hashlib.sha256(lg.tobytes()).digest(), np.uint8))

    record(logits)
    t0 = time.time()
    for i in range(N_GEN):
        t = int(np.argmax(logits))  # first maximum, as sample_greedy
        ids.append(t)
        logits = model.decode(t)
        record(logits)
        if (i + 1) % 32 == 0:
            log(f"decode {i + 1}/{N_GEN}: {time.time() - t0:.1f}s")
    return np.array(ids, np.int32), np.stack(top_i), np.stack(top_v), np.stack(shas)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=8)
    args = ap.parse_args()

    def log(msg):
        print(msg, flush=True)

    pkg = __graft_entry__.load_package()
    info = pkg.synth_preset_info(PRESET)
    prompt = pkg.synth_prompt(info["seed"], N_PROMPT, info["n_vocab"])
    with tempfile.TemporaryDirectory() as td:
        path = f"{td}/{PRESET}.gguf"
        pkg.synth_write(PRESET, path, threads=args.threads)
        sha = file_sha(path)
        log("reference run")
        ref = RefModel(path, MAX_SEQ, LAYOUT, args.threads)
        ids, top_i, top_v, shas = run(ref, prompt, log)
        ref.close()
        log("oracle run")
        orc = OracleModel(path, MAX_SEQ, LAYOUT, args.threads)
        ids_o, top_io, top_vo, shas_o = run(orc, prompt, log)
        if not (np.array_equal(ids, ids_o) and np.array_equal(shas, shas_o)):
            bad = [i for i in range(len(shas)) if not np.array_equal(shas[i], shas_o[i])]
            raise SystemExit(f"oracle differs from the reference: ids equal {np.array_equal(ids, ids_o)}, "
                             f"steps with different logits {bad[:10]}")
        taps = np.stack([orc.tap(layer) for layer in TAP_LAYERS])
        orc.close()
    np.savez_compressed(OUT, gguf_sha256=np.frombuffer(sha, np.uint8), prompt_seed=np.int64(info["seed"]),
                        n_prompt=np.int32(N_PROMPT), max_seq=np.int32(MAX_SEQ), layout=np.int32(LAYOUT),
                        ids=ids, top_idx=top_i, top_val=top_v, logits_sha256=shas,
                        tap_layers=np.array(TAP_LAYERS, np.int32), taps=taps)
    log(f"wrote {OUT}")


if __name__ == "__main__":
    main()
