"""Writes the golden fixtures of the token loop from the reference itself.

Runs the reference compiled from its own sources (oracle/_ref/libref.so, built by
oracle/Makefile where the reference tree exists) on the seeded synthetic GGUFs of this
build and records, per model and KV layout: the GGUF's sha256, the prompt, the greedy
ids, and per step the sha256 of the fp32 logits and their top-4. Also op-level vectors
(f16 table, dequantized random rows of every format, matmul outputs).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import pathlib
import sys
import tempfile

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import __graft_entry__  # noqa: E402
from oracle.bind import RefModel, greedy_stream, ref_lib  # noqa: E402
from rows import random_rows  # noqa: E402

PRESETS = ["tiny_f32", "tiny_q8", "tiny_mixq4", "tiny_qwen", "tiny_hd128", "small_q8"]
N_GREEDY = 16


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def file_sha(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def main():
    pkg = __graft_entry__.load_package()
    R = ref_lib()
    out = {"source": "reference src/*.cpp compiled by oracle/Makefile (g++ -O3 -mavx2 -mfma -mf16c), --stage v2",
           "models": []}
    with tempfile.TemporaryDirectory() as td:
        for preset in PRESETS:
            path = f"{td}/{preset}.gguf"
            pkg.synth_write(preset, path)
            info = pkg.synth_preset_info(preset)
            prompt = pkg.synth_prompt(info["seed"], 6, info["n_vocab"])
            for layout in (0, 1):
                ids, logits = greedy_stream(RefModel(path, 64, layout, 2), prompt, N_GREEDY)
                out["models"].append({
                    "preset": preset, "layout": layout, "max_seq": 64, "gguf_sha256": file_sha(path),
                    "prompt": prompt.tolist(), "ids": ids.tolist(),
                    "logits_sha256": [sha(l) for l in logits],
                    "top4": [[[int(i), float(l[i])] for i in np.argsort(-l, kind="stable")[:4]] for l in logits],
                })
        # the reference CI corpus on its model shape (test_correctness.cpp:102-121)
        path = f"{td}/tiny_f32.gguf"
        ci = []
        for i in range(20):
            prompt = [1, 3 + (i % 20), 5 + (i * 3) % 30, 7]
            ids, _ = greedy_stream(RefModel(path, 64, 0, 2), np.array(prompt, np.int32), 8)
            ci.append({"prompt": prompt, "ids": ids.tolist()})
        out["ci_prompts"] = ci
    (HERE / "token_loop.json").write_text(json.dumps(out, indent=1) + "\n")

    # op-level vectors
    import ctypes as C
    fp = C.POINTER(C.c_float)
    f16 = np.array([R.ref_f16_to_f32(c) for c in range(65536)], np.float32)
    arrays = {"f16_to_f32": f16}
    rng = np.random.default_rng(2024)
    for t in (0, 1, 2, 3, 8, 14):
        k = 256 if t != 0 else 64
        rows = np.ascontiguousarray(random_rows(rng, t, k, 4))
        deq = np.zeros((4, k), np.float32)
        for r in range(4):
            R.ref_dequant_row(t, np.ascontiguousarray(rows[r]).ctypes.data, k, deq[r].ctypes.data_as(fp))
        x = rng.standard_normal((2, k)).astype(np.float32)
        y = np.zeros((2, 4), np.float32)
        R.ref_matmul(y.ctypes.data_as(fp), x.ctypes.data_as(fp), 2, t, rows.ctypes.data, 4, k, 1)
        arrays[f"rows_{t}"] = rows
        arrays[f"dequant_{t}"] = deq
        arrays[f"x_{t}"] = x
        arrays[f"matmul_{t}"] = y
    np.savez_compressed(HERE / "ops.npz", **arrays)
    print(f"wrote {HERE / 'token_loop.json'} and {HERE / 'ops.npz'}")


if __name__ == "__main__":
    main()
