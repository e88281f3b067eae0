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
