"""The library's inline asm keeps the wait states gfx950 requires around it.

hipcc's hazard recognizer pads between compiled instructions only; an inline asm block is
opaque to it.  A v_mul_legacy_f32 in asm that read a v_exp_f32 result in the next cycle
(one wait state required) read the register's old contents, which turned masked rows of a
q8_0 decode tile into NaN in builds whose schedule put the two side by side.  These tests
compile every HIP source of the library to device assembly with the library's own flags
and require that no kernel places an asm instruction closer to its producers or consumers
than gfx950 allows (tests/asm_hazards.py lists the rules).  CPU only: hipcc
cross-compiles.
"""
import importlib.util
import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

import asm_hazards as H

# qubivex_amd/build.py by path: importing the package would load libqvkv.so at collection,
# before torch has set up the HIP runtime that the library must share with it.
_spec = importlib.util.spec_from_file_location(
    "qvkv_build", os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                               "qubivex_amd", "build.py"))
B = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(B)

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not installed")


def _snippet(body):
    return "_Zk:\n" + body + "\n.Lfunc_end0:\n"


@pytest.mark.parametrize("kind,body", [
    ("trans->asm", "v_exp_f32_e32 v95, v95\n;;#ASMSTART\nv_mul_legacy_f32 v97, v95, v97\n;;#ASMEND"),
    ("asm->mfma", ";;#ASMSTART\nv_cvt_f16_i16_sdwa v12, sext(v3) dst_sel:WORD_0 "
     "dst_unused:UNUSED_PAD src0_sel:BYTE_0\ns_nop 0\n;;#ASMEND\n"
     "v_mfma_f32_16x16x16_f16 v[0:3], v[12:13], v[4:5], v[0:3]"),
    ("mfma->asm", "v_mfma_f32_16x16x16_f16 v[0:3], v[12:13], v[4:5], 0\ns_nop 3\n;;#ASMSTART\n"
     "v_mul_legacy_f32 v20, v1, v21\n;;#ASMEND"),
    ("asm-srcc-war", "v_mfma_f32_16x16x16_f16 v[0:3], v[12:13], v[4:5], v[8:11]\n;;#ASMSTART\n"
     "v_cvt_f16_i16_sdwa v8, sext(v30) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n"
     ";;#ASMEND"),
    ("asm-dstsel->valu", ";;#ASMSTART\nv_fma_mixhi_f16 v7, v1, v2, v3 op_sel:[1,0,0] "
     "op_sel_hi:[1,0,0]\n;;#ASMEND\nv_add_f32_e32 v9, v7, v8"),
])
def test_checker_finds_each_hazard(kind, body):
    """Positive controls: each rule fires on a minimal sequence that breaks it, and the
    same sequence padded with enough wait states passes."""
    found = H.check_asm(_snippet(body))
    assert [f.kind for f in found] == [kind], found
    padded = body.replace(";;#ASMSTART\n", ";;#ASMSTART\ns_nop 7\ns_nop 7\n", 1) \
        if kind != "asm-dstsel->valu" and kind != "asm->mfma" else \
        body.replace(";;#ASMEND\n", ";;#ASMEND\ns_nop 7\n")
    assert H.check_asm(_snippet(padded)) == []


def test_compiler_pads_its_own_transcendental_consumers():
    """The checker reads compiled consumers as safe: the exp result read by a compiled
    multiply one instruction later is the compiler's business, not an asm hazard."""
    body = "v_exp_f32_e32 v95, v95\nv_mul_f32_e32 v97, v95, v97"
    assert H.check_asm(_snippet(body)) == []


def _device_asm(src, out_dir):
    out = os.path.join(out_dir, src + ".s")
    subprocess.run(B.hip_command(src, ["--cuda-device-only", "-S"], out), check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    with open(out) as f:
        return f.read()


@pytest.fixture(scope="module")
def texts():
    with tempfile.TemporaryDirectory() as d:
        with ThreadPoolExecutor(len(B.HIP_SOURCES)) as ex:
            return dict(zip(B.HIP_SOURCES, ex.map(lambda s: _device_asm(s, d), B.HIP_SOURCES)))


def test_library_kernels_keep_inline_asm_wait_states(texts):
    n_kernels = 0
    bad = []
    for src, text in texts.items():
        ks = H.kernels(text)
        n_kernels += len(ks)
        bad += [(src,) + tuple(f) for f in H.check_asm(text)]
    assert n_kernels > 50  # every attention, prefill, prelude, append and gather build
    assert bad == [], "\n".join(map(str, bad[:20]))


def test_no_kernel_uses_flat_memory_instructions(texts):
    """Every global access names its address space.  A pointer the compiler cannot place
    (kept in an array, or chosen by a condition) turns its accesses into flat ones, which
    also count on the LDS counter, so LDS waits wait for them too; it once did for every
    output store of the q8_0 gather and append."""
    bad = []
    for src, text in texts.items():
        for name, lines in H.kernels(text).items():
            n = sum(1 for ln in lines if ln.strip().startswith("flat_"))
            if n:
                bad.append((src, name, n))
    assert bad == [], bad
