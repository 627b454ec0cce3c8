"""The oracle against the committed golden fixtures made from the reference
(tests/golden/make_golden.py). These hold without the reference tree: they pin the
oracle bit for bit (sha256 of every step's fp32 logits) on each model and KV layout."""
import ctypes as C
import hashlib
import json
import pathlib

import numpy as np
import pytest

from conftest import n_threads
from oracle.bind import OracleModel, greedy_stream, oracle_lib

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
DATA = json.loads((GOLDEN / "token_loop.json").read_text())


def file_sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


@pytest.mark.parametrize("case", DATA["models"], ids=lambda c: f"{c['preset']}-{c['layout']}")
def test_oracle_reproduces_reference_stream(gguf, case):
    path = gguf(case["preset"])
    assert file_sha(path) == case["gguf_sha256"], "synthetic writer output changed"
    ids, logits = greedy_stream(OracleModel(path, case["max_seq"], case["layout"], n_threads()),
                                np.array(case["prompt"], np.int32), len(case["ids"]))
    assert ids.tolist() == case["ids"]
    for step, (l, want) in enumerate(zip(logits, case["logits_sha256"])):
        assert hashlib.sha256(l.tobytes()).hexdigest() == want, f"step {step}"
        top = np.argsort(-l, kind="stable")[:4]
        assert [[int(i), float(l[i])] for i in top] == case["top4"][step]


def test_oracle_reproduces_reference_ci_corpus(gguf):
    path = gguf("tiny_f32")
    for case in DATA["ci_prompts"]:
        ids, _ = greedy_stream(OracleModel(path, 64, 0, 2), np.array(case["prompt"], np.int32), len(case["ids"]))
        assert ids.tolist() == case["ids"]


def test_oracle_ops_match_golden_vectors():
    ops = np.load(GOLDEN / "ops.npz")
    L = oracle_lib()
    fp = C.POINTER(C.c_float)
    f16 = np.array([L.orc_f16_to_f32(c) for c in range(65536)], np.float32)
    want = ops["f16_to_f32"]
    same = (f16.view(np.uint32) == want.view(np.uint32)) | (np.isnan(f16) & np.isnan(want))
    assert same.all()
    for t in (0, 1, 2, 3, 8, 14):
        rows, deq, x, y = ops[f"rows_{t}"], ops[f"dequant_{t}"], ops[f"x_{t}"], ops[f"matmul_{t}"]
        k = deq.shape[1]
        got = np.zeros_like(deq)
        for r in range(rows.shape[0]):
            L.orc_dequant_row(t, np.ascontiguousarray(rows[r]).ctypes.data, k, got[r].ctypes.data_as(fp))
        assert np.array_equal(got.view(np.uint32), deq.view(np.uint32)), t
        gy = np.zeros_like(y)
        L.orc_matmul(gy.ctypes.data_as(fp), np.ascontiguousarray(x).ctypes.data_as(fp), x.shape[0], t,
                     np.ascontiguousarray(rows).ctypes.data, rows.shape[0], k, 1)
        assert np.array_equal(gy.view(np.uint32), y.view(np.uint32)), t
