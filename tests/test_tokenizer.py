"""The host tokenizer (agent-serve_amd/host/tokenizer.cpp) against the reference's Tokenizer
(tokenizer.cpp:43-239), compiled from its own sources into oracle/_ref: the same ids for
the same text and vocabulary, and the same bytes back.

The vocabularies are byte-level BPE trained here on a small corpus (GPT-2's byte table,
merges by pair frequency), written as metadata-only GGUF files; some merged symbols are
left out of the vocabulary so that the byte fallback runs, and a few entries hold
characters outside the byte table (3- and 4-byte UTF-8)."""
import ctypes as C
import struct

import numpy as np
import pytest

from oracle.bind import ref_available, ref_lib

needs_ref = pytest.mark.skipif(not ref_available(), reason="reference not compiled (oracle/_ref)")

CORPUS = ("the quick brown fox jumps over the lazy dog while the other dogs sleep in the sun "
          "tokenizers split text into pieces and merge frequent pairs of symbols into new symbols "
          "numbers like 2024 and 31337 stay digits it's don't we'll O'Brien rock'n'roll "
          "naïve café über façade déjà vu résumé 日本語 テキスト").split()
SPECIALS = ["<|begin_of_text|>", "<|end_of_text|>", "<|eot_id|>", "<s>", "</s>", "<unk>"]


def byte_chars():
    """GPT-2's table: printable bytes stand for themselves, the others for 256, 257, ..."""
    keep = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    out, extra = {}, 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + extra)
            extra += 1
    return out


def train(n_merges, seed):
    rng = np.random.default_rng(seed)
    bc = byte_chars()
    words = {}
    for w in CORPUS:
        for form in (w, " " + w):
            key = tuple(bc[b] for b in form.encode())
            words[key] = words.get(key, 0) + int(rng.integers(1, 5))
    merges = []
    for _ in range(n_merges):
        pairs = {}
        for w, f in words.items():
            for a, b in zip(w, w[1:]):
                pairs[(a, b)] = pairs.get((a, b), 0) + f
        if not pairs:
            break
        best = min(pairs, key=lambda p: (-pairs[p], p))
        merges.append(best)
        nw = {}
        for w, f in words.items():
            out, i = [], 0
            while i < len(w):
                if i + 1 < len(w) and (w[i], w[i + 1]) == best:
                    out.append(w[i] + w[i + 1])
                    i += 2
                else:
                    out.append(w[i])
                    i += 1
            nw[tuple(out)] = nw.get(tuple(out), 0) + f
        words = nw
    vocab = list(SPECIALS) + [bc[b] for b in range(256)]
    for k, (a, b) in enumerate(merges):
        if k % 7 != 3:  # every 7th merged symbol is missing: its pieces fall back to bytes
            vocab.append(a + b)
    vocab += ["日", "本", "語", "😀", "hello", "<not special"]
    return vocab, [f"{a} {b}" for a, b in merges]


def write_vocab_gguf(path, vocab, merges, bos, eos, add_bos):
    def s(x):
        b = x.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    kv = []
    kv.append(s("general.architecture") + struct.pack("<I", 8) + s("llama"))
    kv.append(s("tokenizer.ggml.model") + struct.pack("<I", 8) + s("gpt2"))
    kv.append(s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, len(vocab)) + b"".join(s(v) for v in vocab))
    kv.append(s("tokenizer.ggml.merges") + struct.pack("<IIQ", 9, 8, len(merges)) + b"".join(s(m) for m in merges))
    kv.append(s("tokenizer.ggml.bos_token_id") + struct.pack("<II", 4, bos))
    kv.append(s("tokenizer.ggml.eos_token_id") + struct.pack("<II", 4, eos))
    if add_bos is not None:
        kv.append(s("tokenizer.ggml.add_bos_token") + struct.pack("<IB", 7, 1 if add_bos else 0))
    with open(path, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, len(kv)) + b"".join(kv))


def random_text(rng, n_words):
    parts = []
    for _ in range(n_words):
        k = rng.integers(0, 12)
        if k < 6:
            parts.append(str(rng.choice(CORPUS)))
        elif k == 6:
            parts.append(str(rng.integers(0, 100000)))
        elif k == 7:
            parts.append(str(rng.choice(SPECIALS + ["<|", "|>", "<>", "<x>"])))
        elif k == 8:
            parts.append(str(rng.choice([",", ".", "!", "?", "'", "--", "(", ")", "'s", "😀", "é", " "])))
        elif k == 9:
            parts.append(str(rng.choice(["  ", "\t", "\n", " \n ", "   "])))
        else:
            parts.append(str(rng.choice(CORPUS)).upper())
        parts.append(str(rng.choice([" ", "", " ", "  "])))
    return "".join(parts)


@pytest.fixture(scope="module")
def vocabs(tmp_path_factory):
    out = []
    for i, (n_merges, add_bos) in enumerate([(300, None), (120, False), (0, True)]):
        vocab, merges = train(n_merges, 11 + i)
        path = tmp_path_factory.mktemp("tok") / f"vocab{i}.gguf"
        write_vocab_gguf(path, vocab, merges, bos=0, eos=1, add_bos=add_bos)
        out.append(str(path))
    return out


def ref_encode(path, text, add_bos):
    cap = 4 * len(text) + 8
    out = np.zeros(cap, np.int32)
    n = ref_lib().ref_tokenize(path.encode(), text, int(add_bos), out.ctypes.data_as(C.POINTER(C.c_int32)), cap)
    assert n >= 0
    return out[:n]


def ref_decode(path, ids):
    ids = np.ascontiguousarray(ids, np.int32)
    cap = 64 * len(ids) + 16
    buf = C.create_string_buffer(cap)
    n = ref_lib().ref_detokenize(path.encode(), ids.ctypes.data_as(C.POINTER(C.c_int32)), len(ids), buf, cap)
    assert n >= 0
    return buf.raw[:n]


def test_known_encodings(pkg, vocabs):
    """Closed cases on the byte-only vocabulary (no merges): one id per byte, after the
    whitespace rule; a special token is one id; BOS first."""
    path = vocabs[2]
    base = len(SPECIALS)  # byte b has id base + b
    ids = pkg.tokenize(path, b"ab", True)
    assert ids.tolist() == [0, base + ord("a"), base + ord("b")]
    # "a  b": the run of two spaces keeps its last space, glued to "b"
    assert pkg.tokenize(path, b"a  b", False).tolist() == [base + ord("a"), base + 32, base + ord("b")]
    assert pkg.tokenize(path, "x<|eot_id|>y".encode(), False).tolist() == [base + ord("x"), 2, base + ord("y")]
    assert pkg.tokenize(path, b"", False).tolist() == []
    assert pkg.detokenize(path, [base + b for b in b"hi there"]) == b"hi there"


@needs_ref
@pytest.mark.parametrize("which", [0, 1, 2])
def test_encode_matches_reference(pkg, vocabs, which):
    path = vocabs[which]
    rng = np.random.default_rng(which)
    texts = ["", " ", "hello", " hello world", "the  quick\tbrown\n\nfox", "it's 2024!", "日本語のテキスト",
             "<|begin_of_text|>hi<|eot_id|>", "<not special>", "a😀b", "  leading and trailing  "]
    texts += [random_text(rng, int(rng.integers(1, 40))) for _ in range(150)]
    for t in texts:
        b = t.encode("utf-8")
        for add_bos in (True, False):
            got = pkg.tokenize(path, b, add_bos)
            want = ref_encode(path, b, add_bos)
            assert got.tolist() == want.tolist(), (t, add_bos)


@needs_ref
@pytest.mark.parametrize("which", [0, 1])
def test_decode_matches_reference(pkg, vocabs, which):
    path = vocabs[which]
    rng = np.random.default_rng(100 + which)
    n_vocab = len(train(300 if which == 0 else 120, 11 + which)[0])
    for _ in range(100):
        ids = rng.integers(-2, n_vocab + 2, int(rng.integers(1, 30)))
        assert pkg.detokenize(path, ids) == ref_decode(path, ids)
    # and round trips of encoded text
    for _ in range(50):
        t = random_text(rng, 20).encode("utf-8")
        ids = pkg.tokenize(path, t, False)
        assert pkg.detokenize(path, ids) == ref_decode(path, ids)
