"""The run-time backend switch as built code: oracle/backend_patch.py applies the change
INTEGRATION.md describes (`--backend hip`, Model forwarding to tf_hip_*) to a copy of the
reference's sources, compiles it with the reference's flags and links libtf_hip.so
(oracle/_ref/tinferno_backend). Here, without a GPU: it links and loads, its CPU path is
the reference's, and `--backend hip` fails cleanly where no GPU exists. The GPU run of the
same binary is in test_gpu_model.py."""
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PATCHED = ROOT / "oracle" / "_ref" / "tinferno_backend"
REFCLI = ROOT / "oracle" / "_ref" / "tinferno"
needs = pytest.mark.skipif(not PATCHED.exists() or not REFCLI.exists(), reason="reference not compiled (oracle/_ref)")


def cli(exe, *args):
    return subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=300)


@needs
def test_patched_reference_links_and_keeps_its_cpu_path(pkg, gguf):
    path = gguf("tiny_q8")
    info = pkg.synth_preset_info("tiny_q8")
    toks = ",".join(str(t) for t in pkg.synth_prompt(info["seed"], 6, info["n_vocab"]))
    args = ["--model", path, "--tokens", toks, "--n-predict", "8", "--max-seq", "64", "--threads", "2"]
    a, b = cli(PATCHED, *args), cli(REFCLI, *args)
    assert a.returncode == 0 and b.returncode == 0, a.stderr + b.stderr
    assert a.stdout == b.stdout and a.stdout.strip()
    assert "--backend" in cli(PATCHED, "--help").stderr


@needs
def test_patched_reference_rejects_bad_backend():
    r = cli(PATCHED, "--model", "x.gguf", "--backend", "tpu", "--tokens", "1")
    assert r.returncode != 0 and "--backend takes cpu or hip" in r.stderr


@needs
def test_patched_reference_without_gpu_fails_cleanly(pkg, gguf):
    import torch  # noqa: F401  (device probe only)
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the GPU test covers this binary")
    r = cli(PATCHED, "--model", gguf("tiny_q8"), "--tokens", "1,2", "--backend", "hip", "--max-seq", "64")
    assert r.returncode != 0 and "tf_hip_create failed" in r.stderr
