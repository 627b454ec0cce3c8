"""Temperature / nucleus sampling on the GPU (tf_hip_sample_logits, tf_hip_sample) against
the oracle's sample_logits (sampler.cpp:15-52), which tests/test_oracle.py pins to the
compiled reference. Same draw r -> the same token; the sorted order and the final
probabilities bit for bit (the device uses the reference libm's expf and sums in sorted
order). Logits are distinct, so the order of ties (unspecified in the reference) does not
arise."""
import ctypes as C

import numpy as np
import pytest

from oracle.bind import oracle_lib

pytestmark = pytest.mark.gpu

F = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))  # noqa: E731
I = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))  # noqa: E731


def oracle_sample(logits, temp, top_p, r):
    L = oracle_lib()
    n = len(logits)
    idx = np.zeros(n, np.int32)
    p = np.zeros(n, np.float32)
    last = np.zeros(1, np.int32)
    tok = L.orc_sample_logits(F(logits), n, temp, top_p, r, I(idx), F(p), I(last))
    return tok, idx, p, int(last[0])


def draws(seed, n):
    out = np.zeros(n, np.float32)
    oracle_lib().orc_uniform_draws(seed, n, F(out))
    return out


def distinct_logits(rng, n, scale):
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    _, first = np.unique(x, return_index=True)
    keep = np.zeros(n, bool)
    keep[first] = True
    x[~keep] = np.float32(scale * 50) + np.arange((~keep).sum(), dtype=np.float32)  # no ties
    return x


CASES = [  # vocab, logit scale, temperature, top_p
    (7, 1.0, 1.0, 1.0), (64, 3.0, 0.7, 0.9), (1000, 0.05, 1.0, 0.9), (4096, 2.0, 1.3, 0.5),
    (32000, 0.02, 0.8, 0.95), (128256, 0.02, 1.0, 0.9), (151936, 1.0, 1.0, 0.9), (151936, 4.0, 0.6, 1.0),
]


@pytest.mark.parametrize("n,scale,temp,top_p", CASES)
def test_sample_logits_matches_oracle(pkg, n, scale, temp, top_p):
    rng = np.random.default_rng(n + int(scale * 100))
    x = distinct_logits(rng, n, scale)
    rs = draws(77 + n, 12)
    for k, r in enumerate(rs):
        r = float(r)
        want, widx, wp, wlast = oracle_sample(x, temp, top_p, r)
        if k < 2:
            tok, idx, p = pkg.sample_logits(x, temp, top_p, r, details=True)
            assert np.array_equal(idx, widx)
            assert np.array_equal(p.view(np.uint32), wp.view(np.uint32)), "probabilities differ"
        else:
            tok = pkg.sample_logits(x, temp, top_p, r)
        assert tok == want, (k, r)


def test_sample_edges(pkg):
    """Draw 0 takes the most likely token, a draw just below 1 the last of the nucleus;
    temperature 0 is the first maximum; two tokens in closed form (3/4, 1/4)."""
    rng = np.random.default_rng(5)
    x = distinct_logits(rng, 5000, 1.0)
    order = np.argsort(-x, kind="stable")
    assert pkg.sample_logits(x, 1.0, 0.9, 0.0) == int(order[0])
    r_hi = float(np.nextafter(np.float32(1), np.float32(0)))
    for top_p in (1.0, 0.9, 0.3):
        assert pkg.sample_logits(x, 1.0, top_p, r_hi) == oracle_sample(x, 1.0, top_p, r_hi)[0]
    assert pkg.sample_logits(x, 0.0, 0.9, 0.5) == int(np.argmax(x))
    two = np.array([0.0, np.log(3.0)], np.float32)
    assert pkg.sample_logits(two, 1.0, 1.0, 0.5) == 1 and pkg.sample_logits(two, 1.0, 1.0, 0.9) == 0


def test_sample_expf_over_its_range(pkg):
    """A million distinct exponent arguments in [-104, 0] (temperature 1): every probability
    is the reference's expf divided by the reference's sum, bit for bit."""
    n = 1 << 20
    x = -np.linspace(0.0, 104.0, n, dtype=np.float64).astype(np.float32)
    x = np.unique(x)[::-1].copy()  # distinct, descending
    _, idx, p = pkg.sample_logits(x, 1.0, 1.0, 0.5, details=True)
    _, widx, wp, _ = oracle_sample(x, 1.0, 1.0, 0.5)
    assert np.array_equal(idx, widx)
    assert np.array_equal(p.view(np.uint32), wp.view(np.uint32))


def test_model_sample_from_device_logits(pkg, gguf):
    """tf_hip_sample on the context's own logits after a prefill equals the oracle on the
    same logits (read back from the same step)."""
    path = gguf("tiny_q8")
    info = pkg.synth_preset_info("tiny_q8")
    m = pkg.HipModel(path, max_seq=64)
    with pytest.raises(RuntimeError):
        m.sample(1.0, 0.9, 0.5)  # no step yet
    logits, _ = m.prefill(pkg.synth_prompt(info["seed"], 6, info["n_vocab"]))
    for r in draws(9, 16):
        for temp, top_p in ((1.0, 0.9), (0.7, 1.0), (1.5, 0.5)):
            assert m.sample(temp, top_p, float(r)) == oracle_sample(logits, temp, top_p, float(r))[0]
    assert m.sample(0.0, 0.9, 0.5) == int(np.argmax(logits))
    # sampling leaves the context ready for the next steps: decode the sampled tokens
    for r in draws(10, 4):
        tok = m.sample(0.9, 0.9, float(r))
        logits, _ = m.decode(tok)
        assert m.sample(0.9, 0.9, 0.25) == oracle_sample(logits, 0.9, 0.9, 0.25)[0]
    m.close()


def test_cli_temperature_sampling_is_seeded(pkg, gguf, tmp_path):
    """tinferno_hip --temp samples on the GPU with the reference's generator: the same seed
    gives the same tokens; --temp 0 prints the greedy stream of tf_hip_generate (the
    synthetic vocabulary's pieces are "tok<id>")."""
    import subprocess

    path = gguf("tiny_q8")
    info = pkg.synth_preset_info("tiny_q8")
    prompt = ",".join(str(t) for t in pkg.synth_prompt(info["seed"], 6, info["n_vocab"]))
    exe = str(pkg.BIN_DIR / "tinferno_hip")

    def run(*extra):
        # the graph path: this test process holds the GPU's cooperative-launch resource (its own
        # step-kernel launches), which a second process cannot take at the same time
        out = subprocess.run([exe, "--model", path, "--tokens", prompt, "--n-predict", "12", "--max-seq", "64",
                              "--decode-path", "graph", *extra], capture_output=True, text=True, timeout=120,
                             check=True)
        return out.stdout.strip()

    a, b = run("--temp", "0.9", "--seed", "7"), run("--temp", "0.9", "--seed", "7")
    assert a and a == b
    # greedy: the pieces of the prefill argmax followed by tf_hip_generate's stream
    m = pkg.HipModel(path, max_seq=64)
    _, first = m.prefill(pkg.synth_prompt(info["seed"], 6, info["n_vocab"]))
    ids = [first] + m.generate(11).tolist()
    eos = m.eos
    m.close()
    stop = next((i for i in range(1, len(ids)) if ids[i] == eos), len(ids))  # the CLI stops at eos
    assert run("--temp", "0") == "".join(f"tok{i}" for i in ids[:stop])
