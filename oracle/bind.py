"""ctypes bindings of the CPU checker (test infrastructure only).

``liboracle.so`` is the C restatement of the reference --stage v2 path (oracle.c);
``_ref/libref.so`` is the reference itself compiled from its own sources
(oracle/Makefile). Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg use this module.
"""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

ORACLE_DIR = pathlib.Path(__file__).resolve().parent
_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)

_orc = None
_ref = None


def _f(a):
    return a.ctypes.data_as(_f32p)


def _i(a):
    return a.ctypes.data_as(_i32p)


def oracle_lib() -> C.CDLL:
    global _orc
    if _orc is not None:
        return _orc
    path = ORACLE_DIR / "liboracle.so"
    if not path.exists():
        raise RuntimeError(f"{path} is not built (make -C oracle)")
    L = C.CDLL(str(path))
    vp = C.c_void_p
    sig = {
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_row_nbytes": (C.c_int64, [C.c_int, C.c_int64]),
        "orc_dequant_row": (C.c_int, [C.c_int, vp, C.c_int64, _f32p]),
        "orc_dot_f32": (C.c_float, [_f32p, _f32p, C.c_int]),
        "orc_dot_row": (C.c_float, [C.c_int, _f32p, vp, C.c_int64]),
        "orc_matmul": (C.c_int, [_f32p, _f32p, C.c_int, C.c_int, vp, C.c_int64, C.c_int64, C.c_int]),
        "orc_rmsnorm": (None, [_f32p, _f32p, _f32p, C.c_int, C.c_float]),
        "orc_silu_mul": (None, [_f32p, _f32p, C.c_int]),
        "orc_softmax": (None, [_f32p, C.c_int]),
        "orc_rope_freqs": (None, [_f32p, C.c_int, C.c_float, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float]),
        "orc_rope": (None, [_f32p, C.c_int, C.c_int, C.c_int, _f32p]),
        "orc_attn_decode": (None, [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   _f32p]),
        "orc_attn_prefill": (None, [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, _f32p]),
        "orc_argmax": (C.c_int, [_f32p, C.c_int]),
        "orc_uniform_draws": (None, [C.c_uint32, C.c_int, _f32p]),
        "orc_sample_logits": (C.c_int, [_f32p, C.c_int, C.c_float, C.c_float, C.c_float, _i32p, _f32p, _i32p]),
        "orc_open": (vp, [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_int]),
        "orc_close": (None, [vp]),
        "orc_prefill": (C.c_int, [vp, _i32p, C.c_int, _f32p]),
        "orc_decode": (C.c_int, [vp, C.c_int32, _f32p]),
        "orc_reset": (None, [vp]),
        "orc_info": (None, [vp, _i32p]),
        "orc_rms_eps": (C.c_float, [vp]),
        "orc_tap": (C.c_int, [vp, C.c_int, _f32p]),
        "orc_read_kv": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, C.c_int, _f32p]),
        "orc_last_error": (C.c_char_p, [vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _orc = L
    return L


def ref_available() -> bool:
    return (ORACLE_DIR / "_ref" / "libref.so").exists()


def ref_lib() -> C.CDLL:
    global _ref
    if _ref is not None:
        return _ref
    path = ORACLE_DIR / "_ref" / "libref.so"
    if not path.exists():
        raise RuntimeError(f"{path} is not built (make -C oracle ref, needs the reference sources)")
    L = C.CDLL(str(path))
    vp = C.c_void_p
    sig = {
        "ref_last_error": (C.c_char_p, []),
        "ref_f16_to_f32": (C.c_float, [C.c_uint16]),
        "ref_dequant_row": (C.c_int, [C.c_int, vp, C.c_int64, _f32p]),
        "ref_matmul": (C.c_int, [_f32p, _f32p, C.c_int, C.c_int, vp, C.c_int64, C.c_int64, C.c_int]),
        "ref_dot_f32": (C.c_float, [_f32p, _f32p, C.c_int]),
        "ref_sample_logits_seq": (None, [_f32p, C.c_int, C.c_float, C.c_float, C.c_uint32, C.c_int, _i32p]),
        "ref_uniform_draws": (None, [C.c_uint32, C.c_int, _f32p]),
        "ref_tokenize": (C.c_int32, [C.c_char_p, C.c_char_p, C.c_int32, _i32p, C.c_int32]),
        "ref_detokenize": (C.c_int32, [C.c_char_p, _i32p, C.c_int32, C.c_char_p, C.c_int32]),
        "ref_rmsnorm": (None, [_f32p, _f32p, _f32p, C.c_int, C.c_float]),
        "ref_silu_mul": (None, [_f32p, _f32p, C.c_int]),
        "ref_softmax": (None, [_f32p, C.c_int]),
        "ref_argmax": (C.c_int, [_f32p, C.c_int]),
        "ref_rope_freqs": (None, [_f32p, C.c_int, C.c_float, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float]),
        "ref_rope": (None, [_f32p, C.c_int, C.c_int, C.c_int, _f32p]),
        "ref_attn_decode": (None, [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
        "ref_attn_prefill": (None, [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int]),
        "ref_open": (vp, [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_int]),
        "ref_close": (None, [vp]),
        "ref_prefill": (C.c_int, [vp, _i32p, C.c_int, _f32p]),
        "ref_decode": (C.c_int, [vp, C.c_int32, _f32p]),
        "ref_reset": (None, [vp]),
        "ref_info": (None, [vp, _i32p]),
        "ref_weight_bytes": (C.c_uint64, [vp]),
        "ref_generate": (C.c_int, [vp, _i32p, C.c_int, C.c_int, _i32p, _f64p, _f64p]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _ref = L
    return L


class OracleModel:
    """The restated v2 Model (oracle.c) over a GGUF file."""

    def __init__(self, path, max_seq=512, kv_layout=0, n_threads=8):
        L = oracle_lib()
        self._L = L
        err = C.create_string_buffer(256)
        self._m = L.orc_open(str(path).encode(), max_seq, kv_layout, n_threads, err, 256)
        if not self._m:
            raise RuntimeError(err.value.decode())
        info = np.zeros(10, np.int32)
        L.orc_info(self._m, _i(info))
        (self.n_vocab, self.n_embd, self.n_ff, self.n_layer, self.n_head, self.n_kv_head, self.head_dim, _,
         self.max_seq, self.kv_layout) = (int(v) for v in info)

    def close(self):
        if self._m:
            self._L.orc_close(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self._L.orc_last_error(self._m).decode())

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.zeros(self.n_vocab, np.float32)
        self._check(self._L.orc_prefill(self._m, _i(t), len(t), _f(logits)))
        return logits

    def decode(self, token):
        logits = np.zeros(self.n_vocab, np.float32)
        self._check(self._L.orc_decode(self._m, int(token), _f(logits)))
        return logits

    def reset(self):
        self._L.orc_reset(self._m)

    def tap(self, layer):
        out = np.zeros(self.n_embd, np.float32)
        self._check(self._L.orc_tap(self._m, layer, _f(out)))
        return out

    def read_kv(self, layer, which, pos0, n):
        out = np.zeros((n, self.n_kv_head, self.head_dim), np.float32)
        self._check(self._L.orc_read_kv(self._m, layer, which, pos0, n, _f(out)))
        return out


class RefModel:
    """tinf::Model of the reference (compiled from its sources) through ref_shim.cpp."""

    def __init__(self, path, max_seq=512, kv_layout=-1, n_threads=0, stage="v2"):
        L = ref_lib()
        self._L = L
        self._m = L.ref_open(str(path).encode(), stage.encode(), max_seq, kv_layout, n_threads)
        if not self._m:
            raise RuntimeError(L.ref_last_error().decode())
        info = np.zeros(7, np.int32)
        L.ref_info(self._m, _i(info))
        self.n_vocab, self.n_embd, self.n_layer, _, self.bos, self.eos, self.n_threads = (int(v) for v in info)

    def close(self):
        if self._m:
            self._L.ref_close(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self._L.ref_last_error().decode())

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.zeros(self.n_vocab, np.float32)
        self._check(self._L.ref_prefill(self._m, _i(t), len(t), _f(logits)))
        return logits

    def decode(self, token):
        logits = np.zeros(self.n_vocab, np.float32)
        self._check(self._L.ref_decode(self._m, int(token), _f(logits)))
        return logits

    def reset(self):
        self._L.ref_reset(self._m)

    def generate(self, prompt, n_predict):
        """bench_e2e's once(): reset, prefill, n greedy decodes; returns (ids, prefill_s, decode_s)."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_predict, np.int32)
        ps, ds = C.c_double(0), C.c_double(0)
        self._check(self._L.ref_generate(self._m, _i(p), len(p), n_predict, _i(out), C.byref(ps), C.byref(ds)))
        return out, float(ps.value), float(ds.value)


def greedy_stream(model, prompt, n):
    """Reference token loop (bench_e2e.cpp:38-59): prefill, then n x (argmax, decode).
    Returns the ids and the logits after prefill and after each decode."""
    logits = model.prefill(prompt)
    ids, all_logits = [], [logits]
    for _ in range(n):
        t = int(np.argmax(logits))  # first maximum, as sample_greedy
        ids.append(t)
        logits = model.decode(t)
        all_logits.append(logits)
    return np.array(ids, np.int32), all_logits
