"""The C-ABI library loads and exports every entry point include/qvkv.h declares (no GPU
compute here), and the layout rules hold."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qvkv.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qvkv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ["qvkv_append_async", "qvkv_gather_async", "qvkv_attention_async",
                 "qvkv_block_copy_async", "qvkv_decode_attention", "qvkv_pool_plan_append",
                 "qvkv_pool_compact", "qvkv_seq_fork", "qvkv_prefix_lookup"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    from qubivex_amd import _lib

    for name in declared():
        assert hasattr(_lib.lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (qvkv_\w+)", out))
    assert set(declared()) <= exported


def test_library_holds_gfx950_code():
    from qubivex_amd import _lib

    out = subprocess.run(["strings", "-n", "6", _lib.LIB], capture_output=True, text=True).stdout
    assert "gfx950" in out


def test_block_bytes_and_layout_rules():
    from qubivex_amd import KvLayout, ShapeError, UnsupportedError, _lib

    assert KvLayout("f16", 4, 128, 16).block_bytes == 2 * 16 * 4 * 128 * 2  # 32 KiB
    assert KvLayout("f16", 8, 128, 16).block_bytes == 64 * 1024
    assert KvLayout("q8_0", 8, 128, 16).block_bytes == 2 * 16 * 8 * 128 * 34 // 32  # 34 KiB
    assert KvLayout("f16", 8, 64, 16).block_bytes == 32 * 1024
    for bad in [KvLayout("f16", 4, 128, 8), KvLayout("f16", 4, 100, 16),
                KvLayout("q8_0", 4, 48, 16), KvLayout("f16", 0, 128, 16)]:
        with pytest.raises(ShapeError):
            bad.block_bytes
    out = ctypes.c_uint64()
    rc = _lib.lib.qvkv_block_bytes(ctypes.byref(_lib.Layout(_lib.F32, 4, 128, 16)), ctypes.byref(out))
    assert rc == _lib.E_UNSUPPORTED
    code, msg = _lib.last_error()
    assert code == _lib.E_UNSUPPORTED and "dtype" in msg


def test_open_without_a_device_is_a_device_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from qubivex_amd import DeviceError, HipDevice

    with pytest.raises(DeviceError):
        HipDevice(0)


def _prototypes():
    """name -> number of parameters, from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    protos = {}
    for m in re.finditer(r"\b(qvkv_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        protos[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return protos


def test_ctypes_signatures_match_the_prototypes():
    """The Python binding declares as many arguments as each C prototype takes."""
    from qubivex_amd import _lib

    protos = _prototypes()
    assert set(protos) == set(declared())
    for name, n in protos.items():
        assert len(_lib.SIGNATURES[name][1]) == n, (name, n, len(_lib.SIGNATURES[name][1]))


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_header_compiles_standalone(tmp_path, lang):
    """include/qvkv.h is a plain C header (what bindgen, cgo or a JNI shim would read)."""
    src = tmp_path / ("h.c" if lang == "c" else "h.cpp")
    src.write_text('#include "qvkv.h"\nint main(void) { return 0; }\n')
    cc = ["gcc", "-std=c99"] if lang == "c" else ["g++", "-std=c++11"]
    r = subprocess.run(cc + ["-Wall", "-Werror", "-pedantic", "-fsyntax-only", "-I",
                             os.path.dirname(HEADER), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_a_c_program_links_and_calls_the_library(tmp_path):
    """A C consumer links libqvkv.so and calls a GPU-free entry point through the header:
    the layout size rule and the thread-local error text."""
    from qubivex_amd import _lib

    src = tmp_path / "use.c"
    src.write_text(r'''
#include <stdio.h>
#include <string.h>
#include "qvkv.h"
int main(void) {
    qvkv_layout l = {QVKV_Q8_0, 8, 128, 16};
    uint64_t bytes = 0;
    if (qvkv_block_bytes(&l, &bytes) != QVKV_OK || bytes != 2ull * 16 * 8 * 128 * 34 / 32) return 1;
    qvkv_layout bad = {QVKV_F16, 4, 100, 16};
    if (qvkv_block_bytes(&bad, &bytes) != QVKV_E_SHAPE) return 2;
    char msg[256];
    qvkv_last_error(msg, sizeof msg);
    if (strstr(msg, "shape mismatch") == NULL) return 3;
    puts("ok");
    return 0;
}
''')
    exe = tmp_path / "use"
    libdir = os.path.dirname(_lib.LIB)
    r = subprocess.run(["gcc", "-std=c99", "-I", os.path.dirname(HEADER), str(src), "-L", libdir,
                        "-lqvkv", "-Wl,-rpath," + libdir, "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)


def test_build_rejects_a_library_with_an_undefined_launch_stub(tmp_path):
    """The build's guard against hipcc's host pass dropping a kernel's launch stub: a shared
    library that references an undefined __device_stub__ symbol is refused (and removed),
    one without is accepted."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("qvkv_build",
                                                  os.path.join(ROOT, "qubivex_amd", "build.py"))
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    bad_c = tmp_path / "bad.c"
    bad_c.write_text("extern void _ZN4qvkv22__device_stub__k_demoEv(void);\n"
                     "void launch(void) { _ZN4qvkv22__device_stub__k_demoEv(); }\n")
    good_c = tmp_path / "good.c"
    good_c.write_text("int launch(void) { return 1; }\n")
    for src in (bad_c, good_c):
        subprocess.run(["gcc", "-shared", "-fPIC", str(src), "-o", str(src.with_suffix(".so"))],
                       check=True)
    build._check_stubs(str(good_c.with_suffix(".so")))
    with pytest.raises(RuntimeError, match="undefined kernel launch stubs"):
        build._check_stubs(str(bad_c.with_suffix(".so")))
    assert not bad_c.with_suffix(".so").exists()


def test_launch_knobs_are_set_through_the_api_only(monkeypatch):
    """qvkv_tune sets a knob process-wide, qvkv_tune_reset restores every default, unknown
    names are refused, and the environment has no say (the library reads none)."""
    from qubivex_amd import kv, ShapeError

    kv.tune_reset()
    assert kv.tune_get("attn_full") == 512
    assert kv.tune_get("attn_waves3_q8") == 0
    monkeypatch.setenv("QVKV_ATTN_FULL", "7")
    monkeypatch.setenv("attn_full", "7")
    assert kv.tune_get("attn_full") == 512
    kv.tune("attn_full", 9)
    assert kv.tune_get("attn_full") == 9
    with kv.tuned({"attn_stream": 0, "stream_unit_cost": 40}):
        assert kv.tune_get("attn_stream") == 0 and kv.tune_get("stream_unit_cost") == 40
    assert kv.tune_get("attn_full") == 512 and kv.tune_get("attn_stream") == 1
    with pytest.raises(ShapeError):
        kv.tune("no_such_knob", 1)
    with pytest.raises(ShapeError):
        kv.tune_get("QVKV_ATTN_FULL")
