"""ctypes bindings of the MI355X backend (lib/libtf_hip.so, include/tf_hip.h) and of the
C++ host side (lib/libtinferno.so): the Model API of the reference (model.hpp:24-50)
running its token loop on the GPU, the op-level entry points, and the seeded
synthetic GGUF writer.

The package directory name is not a Python identifier; load it with ``load_package()``
from ``__graft_entry__`` or by path. Nothing here has a CPU fallback: if the built
libraries are missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

import numpy as np

PKG_DIR = pathlib.Path(__file__).resolve().parent
LIB_DIR = PKG_DIR / "lib"
BIN_DIR = PKG_DIR / "bin"

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q8_0, TYPE_Q6_K = 0, 1, 2, 3, 8, 14
KV_SEQ_MAJOR, KV_HEAD_MAJOR = 0, 1
KERNEL_CLASSES = ("embed", "qkv_gemv", "attention", "wo_gemv", "gateup_gemv", "down_gemv", "lmhead_gemv")

_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)
_u32p = C.POINTER(C.c_uint32)
_u64p = C.POINTER(C.c_uint64)

_hip = None
_host = None


def _need(path: pathlib.Path) -> str:
    if not path.exists():
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build() (make -C agent-serve_amd)")
    return str(path)


def hip_lib() -> C.CDLL:
    """libtf_hip.so with argument types for every entry point of include/tf_hip.h."""
    global _hip
    if _hip is not None:
        return _hip
    L = C.CDLL(_need(LIB_DIR / "libtf_hip.so"))
    vp = C.c_void_p
    sig = {
        "tf_hip_create": (C.c_int, [C.c_int, vp, C.POINTER(vp)]),
        "tf_hip_destroy": (C.c_int, [vp]),
        "tf_hip_last_error": (C.c_char_p, [vp]),
        "tf_hip_upload_tensor": (C.c_int, [vp, C.c_int, C.c_int, C.c_int64, C.c_int64, vp, C.c_size_t]),
        "tf_hip_set_rope_table": (C.c_int, [vp, _f32p, _f32p, C.c_int32, C.c_int32]),
        "tf_hip_prefill": (C.c_int, [vp, _i32p, C.c_int32, _f32p, _i32p]),
        "tf_hip_decode": (C.c_int, [vp, C.c_int32, _f32p, _i32p]),
        "tf_hip_generate": (C.c_int, [vp, C.c_int32, _i32p]),
        "tf_hip_reset": (C.c_int, [vp]),
        "tf_hip_set_decode_path": (C.c_int, [vp, C.c_int32]),
        "tf_hip_get_decode_path": (C.c_int, [vp]),
        "tf_hip_set_split_all_from": (C.c_int, [vp, C.c_int32]),
        "tf_hip_set_split_from": (C.c_int, [vp, C.c_int32]),
        "tf_hip_get_step_config": (C.c_int, [vp, _i32p, C.c_int32]),
        "tf_hip_set_exchange_epoch": (C.c_int, [vp, C.c_uint32]),
        "tf_hip_test_refuse_cooperative": (C.c_int, [vp, C.c_int32]),
        "tf_hip_get_hparams": (C.c_int, [vp, C.POINTER(HParams)]),
        "tf_hip_set_prefill_path": (C.c_int, [vp, C.c_int32]),
        "tf_hip_get_prefill_path": (C.c_int, [vp]),
        "tf_hip_get_pos": (C.c_int, [vp]),
        "tf_hip_get_layer_act": (C.c_int, [vp, C.c_int32, _f32p]),
        "tf_hip_read_kv": (C.c_int, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _f32p]),
        "tf_hip_last_timing": (C.c_int, [vp, _f32p, _f32p, _i32p, C.c_char_p, C.c_int32]),
        "tf_hip_profile_generate": (C.c_int, [vp, C.c_int32, _i32p, _f32p, _i32p, _f64p]),
        "tf_hip_kernel_class_name": (C.c_char_p, [C.c_int32]),
        "tf_hip_dequant_rows": (C.c_int, [C.c_int, C.c_int, vp, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _f32p]),
        "tf_hip_matmul": (C.c_int, [C.c_int, C.c_int, vp, C.c_int64, C.c_int64, _f32p, C.c_int32, _f32p]),
        "tf_hip_rmsnorm": (C.c_int, [C.c_int, _f32p, _f32p, C.c_int32, C.c_int32, C.c_float, _f32p]),
        "tf_hip_rope": (C.c_int, [C.c_int, _f32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _f32p, _f32p, C.c_int32]),
        "tf_hip_sample": (C.c_int, [vp, C.c_float, C.c_float, C.c_float, _i32p]),
        "tf_hip_sample_logits": (C.c_int, [C.c_int, _f32p, C.c_int32, C.c_float, C.c_float, C.c_float, _i32p, _i32p,
                                           _f32p]),
        "tf_hip_attn_decode": (C.c_int, [C.c_int, _f32p, _f32p, _f32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                         C.c_int32, C.c_int32, _f32p]),
        "tf_hip_attn_prefill": (C.c_int, [C.c_int, _f32p, _f32p, _f32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                          _f32p]),
        "tf_hip_attn_decode_noalloc": (C.c_int, [C.c_int, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                                 C.c_int32, C.c_int32, vp, vp]),
        "tf_hip_argmax": (C.c_int, [C.c_int, _f32p, C.c_int32, _i32p]),
        "tf_hip_read_stream": (C.c_int, [C.c_int, C.c_size_t, C.c_int32, _f64p, _f64p, _u32p]),
        "tf_hip_copy_stream": (C.c_int, [C.c_int, C.c_size_t, C.c_int32, _f64p, _f64p, _u32p]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _hip = L
    return L


class HParams(C.Structure):
    """tf_hip_hparams (include/tf_hip.h)."""
    _fields_ = [(n, C.c_int32) for n in ("n_vocab", "n_embd", "n_ff", "n_layer", "n_head", "n_kv_head", "head_dim",
                                         "max_seq", "kv_layout")] + [("rms_eps", C.c_float)]


def host_lib() -> C.CDLL:
    """libtinferno.so (C++ host side) with argument types for its C entry points."""
    global _host
    if _host is not None:
        return _host
    hip_lib()
    L = C.CDLL(_need(LIB_DIR / "libtinferno.so"))
    vp = C.c_void_p
    sig = {
        "tfh_global_error": (C.c_char_p, []),
        "tfh_last_error": (C.c_char_p, [vp]),
        "tfh_open": (vp, [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_int]),
        "tfh_close": (None, [vp]),
        "tfh_prefill": (C.c_int, [vp, _i32p, C.c_int32, _f32p, _i32p]),
        "tfh_decode": (C.c_int, [vp, C.c_int32, _f32p, _i32p]),
        "tfh_generate": (C.c_int, [vp, C.c_int32, _i32p]),
        "tfh_reset": (C.c_int, [vp]),
        "tfh_greedy_host": (C.c_int, [vp, C.c_int32, C.c_int32, _i32p]),
        "tfh_info": (C.c_int, [vp, _i32p]),
        "tfh_weight_bytes": (C.c_uint64, [vp]),
        "tfh_decode_bytes": (C.c_double, [vp, C.c_int32]),
        "tfh_layer_act": (C.c_int, [vp, C.c_int32, _f32p]),
        "tfh_read_kv": (C.c_int, [vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _f32p]),
        "tfh_ctx": (vp, [vp]),
        "tfh_synth_write": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int64, C.c_int32, _u64p]),
        "tfh_synth_preset_info": (C.c_int, [C.c_char_p, _i32p]),
        "tfh_synth_prompt": (C.c_int, [C.c_int64, C.c_int32, C.c_int32, _i32p]),
        "tfh_rope_tables": (C.c_int, [C.c_float, C.c_int32, C.c_int32, _f32p, _f32p]),
        "tfh_file_decode_bytes": (C.c_double, [C.c_char_p, C.c_int32]),
        "tfh_file_rope_tables": (C.c_int, [C.c_char_p, C.c_int32, _f32p, _f32p]),
        "tfh_quantize_row": (C.c_int, [C.c_int32, _f32p, C.c_int64, vp]),
        "tfh_gguf_summary": (C.c_int, [C.c_char_p, _u64p, C.c_char_p, C.c_int32]),
        "tfh_tokenize_file": (C.c_int32, [C.c_char_p, C.c_char_p, C.c_int32, _i32p, C.c_int32]),
        "tfh_detokenize_file": (C.c_int32, [C.c_char_p, _i32p, C.c_int32, C.c_char_p, C.c_int32]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _host = L
    return L


def _f(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _i(a: np.ndarray):
    return a.ctypes.data_as(_i32p)


# ---------------------------------------------------------------- synthetic models

def synth_preset_info(preset: str) -> dict:
    out = np.zeros(7, np.int32)
    if host_lib().tfh_synth_preset_info(preset.encode(), _i(out)) != 0:
        raise ValueError(host_lib().tfh_global_error().decode())
    keys = ("n_vocab", "n_embd", "n_ff", "n_layer", "n_head", "n_kv_head", "seed")
    return dict(zip(keys, (int(v) for v in out)))


def synth_write(preset: str, path: str, seed: int = -1, threads: int = 0) -> int:
    """Writes the preset's GGUF to path; returns its weight bytes."""
    wb = C.c_uint64(0)
    if host_lib().tfh_synth_write(preset.encode(), str(path).encode(), seed, threads, C.byref(wb)) != 0:
        raise RuntimeError(host_lib().tfh_global_error().decode())
    return int(wb.value)


def synth_prompt(seed: int, n: int, n_vocab: int) -> np.ndarray:
    out = np.zeros(max(n, 0), np.int32)
    if n > 0 and host_lib().tfh_synth_prompt(seed, n, n_vocab, _i(out)) != 0:
        raise RuntimeError(host_lib().tfh_global_error().decode())
    return out


def quantize_row(ggml_type: int, x: np.ndarray) -> np.ndarray:
    """The synthetic writer's quantizer for one row (GGUF block bytes)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    blk = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34), 14: (256, 210)}[ggml_type]
    out = np.zeros(len(x) // blk[0] * blk[1], np.uint8)
    if host_lib().tfh_quantize_row(ggml_type, _f(x), len(x), out.ctypes.data) != 0:
        raise RuntimeError(host_lib().tfh_global_error().decode())
    return out


def gguf_summary(path: str) -> dict:
    out = np.zeros(3, np.uint64)
    arch = C.create_string_buffer(64)
    if host_lib().tfh_gguf_summary(str(path).encode(), out.ctypes.data_as(_u64p), arch, 64) != 0:
        raise RuntimeError(host_lib().tfh_global_error().decode())
    return {"n_tensors": int(out[0]), "weight_bytes": int(out[1]), "file_size": int(out[2]),
            "arch": arch.value.decode()}


def rope_tables(theta: float, n_rot: int, n_pos: int):
    c = np.zeros((n_pos, n_rot // 2), np.float32)
    s = np.zeros((n_pos, n_rot // 2), np.float32)
    if host_lib().tfh_rope_tables(theta, n_rot, n_pos, _f(c), _f(s)) != 0:
        raise RuntimeError(host_lib().tfh_global_error().decode())
    return c, s


def tokenize(path: str, text: bytes, add_bos: bool = True) -> np.ndarray:
    """Tokenizer::encode (tokenizer.cpp:183-201) of text with the GGUF's vocabulary (host side)."""
    L = host_lib()
    cap = 4 * len(text) + 8
    out = np.zeros(cap, np.int32)
    n = L.tfh_tokenize_file(str(path).encode(), text, int(add_bos), _i(out), cap)
    if n < 0:
        raise RuntimeError(L.tfh_global_error().decode())
    return out[:n].copy()


def detokenize(path: str, ids) -> bytes:
    """Tokenizer::decode (tokenizer.cpp:233-237) with the GGUF's vocabulary (host side)."""
    L = host_lib()
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    cap = 64 * len(ids) + 16
    buf = C.create_string_buffer(cap)
    n = L.tfh_detokenize_file(str(path).encode(), _i(ids), len(ids), buf, cap)
    if n < 0:
        raise RuntimeError(L.tfh_global_error().decode())
    return buf.raw[:n]


def file_decode_bytes(path: str, pos: int) -> float:
    """Algorithmic bytes of one decode step at position pos of the GGUF at path (the
    roofline's numerator, Model::decode_bytes), computed on the host."""
    v = host_lib().tfh_file_decode_bytes(str(path).encode(), int(pos))
    if v < 0:
        raise RuntimeError(host_lib().tfh_global_error().decode())
    return float(v)


def file_rope_tables(path: str, n_pos: int, half_dim: int):
    """The host RoPE cos/sin tables the Model uploads for the GGUF at path."""
    c = np.zeros((n_pos, half_dim), np.float32)
    s = np.zeros((n_pos, half_dim), np.float32)
    if host_lib().tfh_file_rope_tables(str(path).encode(), n_pos, _f(c), _f(s)) != 0:
        raise RuntimeError(host_lib().tfh_global_error().decode())
    return c, s


# ---------------------------------------------------------------- Model on the GPU

class HipModel:
    """Model(path, RunConfig) of model.hpp:24-50 with its token loop on the GPU."""

    def __init__(self, path: str, max_seq: int = 4096, kv_layout: int = -1, stage: str = "v2", device: int = 0):
        L = host_lib()
        self._L = L
        self._h = L.tfh_open(str(path).encode(), stage.encode(), max_seq, kv_layout, device)
        if not self._h:
            raise RuntimeError(L.tfh_global_error().decode())
        info = np.zeros(12, np.int32)
        L.tfh_info(self._h, _i(info))
        (self.n_vocab, self.n_embd, self.n_ff, self.n_layer, self.n_head, self.n_kv_head, self.head_dim, _,
         self.max_seq, self.kv_layout, self.bos, self.eos) = (int(v) for v in info)

    def _check(self, rc: int):
        if rc != 0:
            raise RuntimeError(self._L.tfh_last_error(self._h).decode())

    def close(self):
        if self._h:
            self._L.tfh_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def n_pos(self) -> int:
        info = np.zeros(12, np.int32)
        self._L.tfh_info(self._h, _i(info))
        return int(info[7])

    def prefill(self, tokens, want_logits: bool = True):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.zeros(self.n_vocab, np.float32) if want_logits else None
        am = C.c_int32(-1)
        self._check(self._L.tfh_prefill(self._h, _i(t), len(t), _f(logits) if want_logits else None, C.byref(am)))
        return logits, int(am.value)

    def decode(self, token: int, want_logits: bool = True):
        logits = np.zeros(self.n_vocab, np.float32) if want_logits else None
        am = C.c_int32(-1)
        self._check(self._L.tfh_decode(self._h, int(token), _f(logits) if want_logits else None, C.byref(am)))
        return logits, int(am.value)

    def generate(self, n: int) -> np.ndarray:
        out = np.zeros(n, np.int32)
        self._check(self._L.tfh_generate(self._h, n, _i(out)))
        return out

    def greedy_host(self, first: int, n: int) -> np.ndarray:
        """The drop-in caller's greedy loop (tfh_greedy_host): n decodes, each copying the
        logits to the host and taking their first maximum there; returns the tokens fed."""
        out = np.zeros(n, np.int32)
        self._check(self._L.tfh_greedy_host(self._h, int(first), n, _i(out)))
        return out

    def sample(self, temperature: float, top_p: float, r: float) -> int:
        """sample_logits (sampler.cpp:15-52) of the last step's logits on the GPU for the draw r."""
        tok = np.zeros(1, np.int32)
        rc = hip_lib().tf_hip_sample(self._L.tfh_ctx(self._h), temperature, top_p, r, _i(tok))
        if rc != 0:
            raise RuntimeError(f"tf_hip_sample failed: {rc}")
        return int(tok[0])

    def reset(self):
        self._check(self._L.tfh_reset(self._h))

    PATH_GRAPH, PATH_STEP = 0, 1

    def set_decode_path(self, path: int):
        """PATH_STEP: one persistent kernel per call where the model allows it (default);
        PATH_GRAPH: the captured per-layer graph, replayed per token."""
        H = hip_lib()
        rc = H.tf_hip_set_decode_path(self._L.tfh_ctx(self._h), int(path))
        if rc != 0:
            raise RuntimeError(f"tf_hip_set_decode_path({path}) failed: {rc}")

    def set_split_all_from(self, span: int):
        """Step kernel, caches longer than 512 positions: spans of more than `span` positions
        split attention over every workgroup (span < 0: the model-derived default)."""
        rc = hip_lib().tf_hip_set_split_all_from(self._L.tfh_ctx(self._h), int(span))
        if rc != 0:
            raise RuntimeError(f"tf_hip_set_split_all_from({span}) failed: {rc}")

    def set_split_from(self, span: int):
        """Step kernel: spans of at most `span` positions attend on one workgroup per kv
        head, longer ones split (span < 0: the default, 64; at most 512)."""
        H = hip_lib()
        rc = H.tf_hip_set_split_from(self._L.tfh_ctx(self._h), int(span))
        if rc != 0:
            raise RuntimeError(H.tf_hip_last_error(self._L.tfh_ctx(self._h)).decode())

    def step_config(self) -> dict:
        """The step kernel's attention configuration (raises when the step kernel does not
        run this model)."""
        H = hip_lib()
        out = np.zeros(5, np.int32)
        rc = H.tf_hip_get_step_config(self._L.tfh_ctx(self._h), _i(out), 5)
        if rc != 0:
            raise RuntimeError(H.tf_hip_last_error(self._L.tfh_ctx(self._h)).decode())
        keys = ("n_wg", "split", "split_all", "split_from", "split_all_from")
        return dict(zip(keys, (int(v) for v in out)))

    def set_exchange_epoch(self, epoch: int):
        """Test hook: the step kernel's exchange epoch counter."""
        rc = hip_lib().tf_hip_set_exchange_epoch(self._L.tfh_ctx(self._h), int(epoch) & 0xFFFFFFFF)
        if rc != 0:
            raise RuntimeError(f"tf_hip_set_exchange_epoch failed: {rc}")

    def device_hparams(self) -> dict:
        """The hyperparameters the device context was created with (tf_hip_get_hparams);
        kv_layout is the device KV cache's layout (0 seq-major, 1 head-major)."""
        hp = HParams()
        rc = hip_lib().tf_hip_get_hparams(self._L.tfh_ctx(self._h), C.byref(hp))
        if rc != 0:
            raise RuntimeError(f"tf_hip_get_hparams failed: {rc}")
        return {n: getattr(hp, n) for n, _ in HParams._fields_}

    def test_refuse_cooperative(self, n: int):
        """Test hook: the next n step-kernel launches report a cooperative-launch refusal."""
        rc = hip_lib().tf_hip_test_refuse_cooperative(self._L.tfh_ctx(self._h), int(n))
        if rc != 0:
            raise RuntimeError(f"tf_hip_test_refuse_cooperative failed: {rc}")

    def decode_path(self) -> int:
        H = hip_lib()
        rc = H.tf_hip_get_decode_path(self._L.tfh_ctx(self._h))
        if rc < 0:
            raise RuntimeError(H.tf_hip_last_error(self._L.tfh_ctx(self._h)).decode())
        return rc

    PREFILL_TOKENS, PREFILL_MFMA = 0, 1

    def set_prefill_path(self, path: int):
        """PREFILL_MFMA: prompts of two or more tokens on the matrix cores where the model
        allows it (default); PREFILL_TOKENS: one prompt token at a time on the decode path."""
        H = hip_lib()
        rc = H.tf_hip_set_prefill_path(self._L.tfh_ctx(self._h), int(path))
        if rc != 0:
            raise RuntimeError(f"tf_hip_set_prefill_path({path}) failed: {rc}")

    def prefill_path(self) -> int:
        H = hip_lib()
        rc = H.tf_hip_get_prefill_path(self._L.tfh_ctx(self._h))
        if rc < 0:
            raise RuntimeError(H.tf_hip_last_error(self._L.tfh_ctx(self._h)).decode())
        return rc

    def layer_act(self, layer: int) -> np.ndarray:
        out = np.zeros(self.n_embd, np.float32)
        self._check(self._L.tfh_layer_act(self._h, layer, _f(out)))
        return out

    def read_kv(self, layer: int, which: int, pos0: int, n: int) -> np.ndarray:
        out = np.zeros((n, self.n_kv_head, self.head_dim), np.float32)
        self._check(self._L.tfh_read_kv(self._h, layer, which, pos0, n, _f(out)))
        return out

    def weight_bytes(self) -> int:
        return int(self._L.tfh_weight_bytes(self._h))

    def decode_bytes(self, pos: int) -> float:
        return float(self._L.tfh_decode_bytes(self._h, pos))

    def last_timing(self):
        H = hip_lib()
        tot, k = C.c_float(0), C.c_float(0)
        n = C.c_int32(0)
        name = C.create_string_buffer(64)
        H.tf_hip_last_timing(self._L.tfh_ctx(self._h), C.byref(tot), C.byref(k), C.byref(n), name, 64)
        return float(tot.value), float(k.value), int(n.value), name.value.decode()

    def profile_generate(self, n: int):
        """Per kernel class: (ms, launches, bytes) over n greedy steps launched kernel by kernel."""
        H = hip_lib()
        out = np.zeros(n, np.int32)
        ms = np.zeros(len(KERNEL_CLASSES), np.float32)
        launches = np.zeros(len(KERNEL_CLASSES), np.int32)
        nbytes = np.zeros(len(KERNEL_CLASSES), np.float64)
        rc = H.tf_hip_profile_generate(self._L.tfh_ctx(self._h), n, _i(out), _f(ms), _i(launches),
                                       nbytes.ctypes.data_as(_f64p))
        if rc != 0:
            raise RuntimeError(H.tf_hip_last_error(self._L.tfh_ctx(self._h)).decode())
        return out, {KERNEL_CLASSES[k]: (float(ms[k]), int(launches[k]), float(nbytes[k]))
                     for k in range(len(KERNEL_CLASSES))}


# ---------------------------------------------------------------- op-level entry points

def _op(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what} failed with status {rc}")


def dequant_rows(ggml_type: int, raw: np.ndarray, ne0: int, ne1: int, row0: int = 0, nrows: int | None = None,
                 device: int = 0) -> np.ndarray:
    nrows = ne1 - row0 if nrows is None else nrows
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros((nrows, ne0), np.float32)
    _op(hip_lib().tf_hip_dequant_rows(device, ggml_type, raw.ctypes.data, ne0, ne1, row0, nrows, _f(out)),
        "tf_hip_dequant_rows")
    return out


def matmul(ggml_type: int, raw: np.ndarray, ne0: int, ne1: int, x: np.ndarray, device: int = 0) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    y = np.zeros((x.shape[0], ne1), np.float32)
    _op(hip_lib().tf_hip_matmul(device, ggml_type, raw.ctypes.data, ne0, ne1, _f(x), x.shape[0], _f(y)),
        "tf_hip_matmul")
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, device: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    _op(hip_lib().tf_hip_rmsnorm(device, _f(x), _f(w), x.shape[1], x.shape[0], eps, _f(out)), "tf_hip_rmsnorm")
    return out


def sample_logits(logits: np.ndarray, temperature: float, top_p: float, r: float, device: int = 0,
                  details: bool = False):
    """sample_logits (sampler.cpp:15-52) of host logits on the GPU for the uniform draw r; with
    details, also the sorted order and the final probabilities."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    n = x.shape[0]
    tok = np.zeros(1, np.int32)
    idx = np.zeros(n, np.int32) if details else None
    p = np.zeros(n, np.float32) if details else None
    _op(hip_lib().tf_hip_sample_logits(device, _f(x), n, temperature, top_p, r, _i(tok),
                                       _i(idx) if details else None, _f(p) if details else None),
        "tf_hip_sample_logits")
    return (int(tok[0]), idx, p) if details else int(tok[0])


def rope(x: np.ndarray, pos0: int, cos_tab: np.ndarray, sin_tab: np.ndarray, device: int = 0) -> np.ndarray:
    """apply_rope_many (attention.cpp:48-53) of x [seq][n_heads][head_dim] on the GPU, angles from
    the host tables [n_pos][head_dim/2] (rope_tables); returns the rotated copy."""
    out = np.ascontiguousarray(x, dtype=np.float32).copy()
    seq, n_heads, hd = out.shape
    c = np.ascontiguousarray(cos_tab, dtype=np.float32)
    s = np.ascontiguousarray(sin_tab, dtype=np.float32)
    _op(hip_lib().tf_hip_rope(device, _f(out), seq, n_heads, hd, pos0, _f(c), _f(s), c.shape[0]), "tf_hip_rope")
    return out


def attn_decode(q: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray, max_seq: int, layout: int,
                device: int = 0) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k_rows = np.ascontiguousarray(k_rows, dtype=np.float32)
    v_rows = np.ascontiguousarray(v_rows, dtype=np.float32)
    n_heads, hd = q.shape
    n_pos, n_kv, _ = k_rows.shape
    out = np.zeros_like(q)
    _op(hip_lib().tf_hip_attn_decode(device, _f(q), _f(k_rows), _f(v_rows), n_heads, n_kv, hd, n_pos, max_seq,
                                     layout, _f(out)), "tf_hip_attn_decode")
    return out


def attn_prefill(q: np.ndarray, k: np.ndarray, v: np.ndarray, device: int = 0) -> np.ndarray:
    """attn_prefill (attention.cpp:82-111): q [seq][n_heads][hd], k and v [seq][n_kv][hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    seq, n_heads, hd = q.shape
    n_kv = k.shape[1]
    out = np.zeros_like(q)
    _op(hip_lib().tf_hip_attn_prefill(device, _f(q), _f(k), _f(v), seq, n_heads, n_kv, hd, _f(out)),
        "tf_hip_attn_prefill")
    return out


def argmax(x: np.ndarray, device: int = 0) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = C.c_int32(-1)
    _op(hip_lib().tf_hip_argmax(device, _f(x), len(x), C.byref(out)), "tf_hip_argmax")
    return int(out.value)


def stream_checksum(nbytes: int) -> int:
    """The sum (mod 2^32) of the streams' fill pattern over nbytes (rounded down to 16):
    word i holds i * 0x9E3779B1, so n words sum to 0x9E3779B1 * n (n - 1) / 2."""
    n = nbytes // 16 * 4
    return (0x9E3779B1 * (n * (n - 1) // 2)) % (1 << 32)


def read_stream(nbytes: int, iters: int = 10, device: int = 0, with_checksum: bool = False):
    """Read-only stream over nbytes of device memory: (best GB/s, median GB/s), plus the
    integer sum of every word read when with_checksum."""
    best, med, cs = C.c_double(0), C.c_double(0), C.c_uint32(0)
    _op(hip_lib().tf_hip_read_stream(device, nbytes, iters, C.byref(best), C.byref(med), C.byref(cs)),
        "tf_hip_read_stream")
    r = (float(best.value), float(med.value))
    return r + (int(cs.value),) if with_checksum else r


def copy_stream(nbytes: int, iters: int = 10, device: int = 0, with_checksum: bool = False):
    """Device-to-device copy of nbytes; GB/s counts bytes read plus bytes written. With
    with_checksum also the integer sum of the destination after the copies."""
    best, med, cs = C.c_double(0), C.c_double(0), C.c_uint32(0)
    _op(hip_lib().tf_hip_copy_stream(device, nbytes, iters, C.byref(best), C.byref(med), C.byref(cs)),
        "tf_hip_copy_stream")
    r = (float(best.value), float(med.value))
    return r + (int(cs.value),) if with_checksum else r
