"""The C-ABI libraries load on a machine without a GPU and export every entry point their
headers declare (no compute calls here)."""
import ctypes as C
import pathlib
import re

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared(header: pathlib.Path, prefix: str):
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(rf"\b({prefix}\w+)\s*\(", text)) - {prefix.rstrip("_")})


def test_tf_hip_exports_every_declared_symbol(pkg):
    names = declared(ROOT / "include" / "tf_hip.h", "tf_hip_")
    assert len(names) >= 20
    lib = C.CDLL(str(ROOT / "agent-serve_amd" / "lib" / "libtf_hip.so"))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert "tf_hip_decode" in names and "tf_hip_prefill" in names and "tf_hip_create" in names


def test_host_library_loads(pkg):
    L = pkg.host_lib()
    for n in ("tfh_open", "tfh_prefill", "tfh_decode", "tfh_generate", "tfh_synth_write"):
        assert hasattr(L, n)


def test_oracle_exports(pkg):
    from oracle.bind import oracle_lib
    names = declared(ROOT / "oracle" / "oracle.h", "orc_")
    lib = oracle_lib()
    assert not [n for n in names if not hasattr(lib, n)]


def test_error_status_without_gpu_is_clean(pkg):
    """Null/invalid arguments are rejected before any device work."""
    H = pkg.hip_lib()
    out = C.c_void_p()
    assert H.tf_hip_create(0, None, C.byref(out)) == -1
    assert H.tf_hip_decode(None, 0, None, None) == -1
    assert H.tf_hip_last_error(None) == b"null context"
