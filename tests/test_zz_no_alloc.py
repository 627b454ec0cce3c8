"""The allocation-free decode attention (tf_hip_attn_decode_noalloc) against the existing
entry point tf_hip_attn_decode on the same rows, through the C ABI.

Both run the same kernels with the same split count, so the outputs are compared bit for
bit. The test's device buffers and stream come from the HIP runtime the library itself
links (libamdhip64.so.7, already loaded with it), not from another runtime: the entry point
allocates nothing, and its split partials live in the library's static scratch, shared by
the calls made one after another here.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 4 << 20   # TF_HIP_ATTN_SCRATCH_BYTES
E_SCRATCH = -6            # TF_HIP_ESCRATCH
H2D, D2H = 1, 2           # hipMemcpyHostToDevice, hipMemcpyDeviceToHost


class Hip:
    """The few HIP runtime calls the test needs, from the library's own runtime."""

    def __init__(self, pkg):
        pkg.hip_lib()  # loads libamdhip64.so.7 as the library's dependency
        self.L = C.CDLL("libamdhip64.so.7")
        self.L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.L.hipFree.argtypes = [C.c_void_p]
        self.L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.L.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.L.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.L.hipStreamDestroy.argtypes = [C.c_void_p]
        self.L.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.L.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.L.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        self.L.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.L.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.L.hipGraphDestroy.argtypes = [C.c_void_p]
        assert self.L.hipSetDevice(0) == 0
        self.mem = []

    def upload(self, a):
        a = np.ascontiguousarray(a, np.float32)
        p = C.c_void_p()
        assert self.L.hipMalloc(C.byref(p), max(a.nbytes, 16)) == 0
        self.mem.append(p)
        assert self.L.hipMemcpy(p, a.ctypes.data, a.nbytes, H2D) == 0
        return p

    def download(self, p, shape):
        out = np.zeros(shape, np.float32)
        assert self.L.hipMemcpy(out.ctypes.data, p, out.nbytes, D2H) == 0
        return out

    def close(self):
        for p in self.mem:
            self.L.hipFree(p)
        self.mem = []


def splits(max_seq):
    return 1 if max_seq <= 512 else min(512, max(2, -(-max_seq // 32)))


def cache_of(rows, max_seq, layout):
    """rows [n_pos][n_kv][hd] -> a cache of max_seq positions in the given layout."""
    n_pos, n_kv, hd = rows.shape
    if layout == 0:
        c = np.zeros((max_seq, n_kv, hd), np.float32)
        c[:n_pos] = rows
    else:
        c = np.zeros((n_kv, max_seq, hd), np.float32)
        c[:, :n_pos] = rows.transpose(1, 0, 2)
    return np.ascontiguousarray(c)


def noalloc(pkg, hip, stream, q, k_rows, v_rows, max_seq, layout):
    n_heads, hd = q.shape
    n_pos, n_kv, _ = k_rows.shape
    dq = hip.upload(q)
    dk = hip.upload(cache_of(k_rows, max_seq, layout))
    dv = hip.upload(cache_of(v_rows, max_seq, layout))
    out = hip.upload(np.full(q.shape, np.nan, np.float32))
    rc = pkg.hip_lib().tf_hip_attn_decode_noalloc(0, dq, dk, dv, n_heads, n_kv, hd, n_pos, max_seq, layout, out,
                                                  stream)
    assert hip.L.hipStreamSynchronize(stream) == 0
    return rc, hip.download(out, q.shape)


# n_heads, n_kv, hd, n_pos, max_seq, layout: a long cache (47 splits of the 2048-position
# cache, Llama-3.2-1B heads), then a smaller one (Qwen2.5-1.5B heads, head-major), then a
# cache of at most 512 positions (one split, no partials)
CASES = [(32, 8, 64, 1500, 2048, 0), (12, 2, 128, 700, 1024, 1), (14, 2, 64, 300, 512, 0)]


def test_noalloc_attention_matches_existing_entry_point(pkg):
    hip = Hip(pkg)
    stream = C.c_void_p()
    assert hip.L.hipStreamCreate(C.byref(stream)) == 0
    rng = np.random.default_rng(97)
    try:
        for n_heads, n_kv, hd, n_pos, max_seq, layout in CASES:
            assert n_heads * splits(max_seq) * (hd + 2) * 4 <= SCRATCH_BYTES
            q = rng.standard_normal((n_heads, hd)).astype(np.float32)
            k = rng.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
            v = rng.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
            want = pkg.attn_decode(q, k, v, max_seq, layout)
            rc, got = noalloc(pkg, hip, stream, q, k, v, max_seq, layout)
            assert rc == 0
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n_heads, n_kv, hd, n_pos, max_seq)
    finally:
        hip.L.hipStreamSynchronize(stream)
        hip.L.hipStreamDestroy(stream)
        hip.close()


def test_noalloc_attention_rejects_requests_past_its_scratch(pkg):
    """64 heads of 128 over a 16384-position cache need 512 splits x 64 x 130 x 4 bytes
    (17 MB) of partials: refused before any launch (the pointers are never used)."""
    n_heads, n_kv, hd, max_seq = 64, 8, 128, 16384
    assert n_heads * splits(max_seq) * (hd + 2) * 4 > SCRATCH_BYTES
    hip = Hip(pkg)
    try:
        buf = hip.upload(np.zeros(16, np.float32))
        rc = pkg.hip_lib().tf_hip_attn_decode_noalloc(0, buf, buf, buf, n_heads, n_kv, hd, 100, max_seq, 0, buf,
                                                      None)
        assert rc == E_SCRATCH
    finally:
        hip.close()


CAPTURE_GLOBAL = 0  # hipStreamCaptureModeGlobal


def test_noalloc_attention_under_graph_capture(pkg):
    """After a warm-up call outside capture (the first call on a device looks up the
    scratch's address), the entry point is captured into a graph on a caller's stream; each
    replay, with the output cleared and other calls rewriting the shared scratch in between,
    gives tf_hip_attn_decode's result bit for bit."""
    n_heads, n_kv, hd, n_pos, max_seq, layout = CASES[0]
    hip = Hip(pkg)
    stream = C.c_void_p()
    assert hip.L.hipStreamCreate(C.byref(stream)) == 0
    graph, gexec = C.c_void_p(), C.c_void_p()
    rng = np.random.default_rng(131)
    lib = pkg.hip_lib()
    try:
        q = rng.standard_normal((n_heads, hd)).astype(np.float32)
        k = rng.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
        v = rng.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
        want = pkg.attn_decode(q, k, v, max_seq, layout)
        dq = hip.upload(q)
        dk = hip.upload(cache_of(k, max_seq, layout))
        dv = hip.upload(cache_of(v, max_seq, layout))
        out = hip.upload(np.full(q.shape, np.nan, np.float32))
        q2 = hip.upload(rng.standard_normal((n_heads, hd)).astype(np.float32))
        out2 = hip.upload(np.zeros(q.shape, np.float32))

        def call(qp, op):
            return lib.tf_hip_attn_decode_noalloc(0, qp, dk, dv, n_heads, n_kv, hd, n_pos, max_seq, layout, op,
                                                 stream)

        assert call(dq, out) == 0  # warm-up, outside capture
        assert hip.L.hipStreamSynchronize(stream) == 0
        assert np.array_equal(hip.download(out, q.shape).view(np.uint32), want.view(np.uint32))

        assert hip.L.hipStreamBeginCapture(stream, CAPTURE_GLOBAL) == 0
        rc = call(dq, out)
        assert hip.L.hipStreamEndCapture(stream, C.byref(graph)) == 0
        assert rc == 0
        assert hip.L.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0) == 0
        nan = np.full(q.shape, np.nan, np.float32)
        for replay in range(3):
            assert hip.L.hipMemcpy(out, nan.ctypes.data, nan.nbytes, H2D) == 0
            assert hip.L.hipGraphLaunch(gexec, stream) == 0
            assert hip.L.hipStreamSynchronize(stream) == 0
            got = hip.download(out, q.shape)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), replay
            assert call(q2, out2) == 0  # eager work between replays rewrites the scratch
            assert hip.L.hipStreamSynchronize(stream) == 0
    finally:
        hip.L.hipStreamSynchronize(stream)
        if gexec.value:
            hip.L.hipGraphExecDestroy(gexec)
        if graph.value:
            hip.L.hipGraphDestroy(graph)
        hip.L.hipStreamDestroy(stream)
        hip.close()
