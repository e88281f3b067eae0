"""Static check of the hazards that inline asm hides from the compiler (gfx950).

LLVM's hazard recognizer inserts the wait states gfx950 needs between its own
instructions, but treats an inline asm statement as opaque: it neither pads after an
asm block for the next instruction nor before one for what the block reads.  The
library's kernels use inline asm for the int8 -> f16 SDWA conversions, the f16
high/residual splits (v_fma_mixlo/mixhi_f16) and v_mul_legacy_f32.  This module reads
the device assembly hipcc writes for a source file (`-S --cuda-device-only`) and reports,
per kernel, every place where an instruction inside an asm block and an instruction
around it are closer than gfx950 allows:

* ``trans->asm``: an asm instruction reads a VGPR that a transcendental instruction
  (v_exp/v_log/v_rcp/v_rsq/v_sqrt/v_sin/v_cos) wrote in the previous wait state (gfx940
  family: 1 wait state before a non-transcendental VALU consumer);
* ``asm->mfma``: an MFMA reads a VGPR that an asm instruction wrote less than 2 wait
  states before;
* ``mfma->asm``: an asm instruction reads or writes a VGPR that an MFMA is still writing
  (fewer than ``raw`` wait states since the MFMA issued -- the compiler's own reads come 8
  or more after a 16x16 f16 MFMA; 12 is on the safe side -- and no compiled instruction has
  touched the register since, which would have made the compiler wait);
* ``asm-srcc-war``: an asm instruction overwrites the SrcC accumulator of an MFMA still in
  flight (fewer than ``war`` wait states after it; the compiler's own code places such
  writes 3 wait states after a v_mfma_f32_16x16x16_f16, so 4 is on the safe side);
* ``asm-dstsel->valu``: a compiled VALU instruction reads, in the next wait state, a VGPR
  that an asm SDWA instruction (dst_sel) or a hi-half op_sel write produced.

Wait states are counted as instructions, ``s_nop n`` as n + 1.  The scan is linear in
program order (fall-through), which is where the asm blocks and their producers and
consumers sit in these kernels.
"""
import re
from collections import namedtuple

Finding = namedtuple("Finding", "kind kernel wait_states producer consumer")

TRANS = re.compile(r"^v_(exp|log|rcp|rsq|sqrt|sin|cos)_")
_RANGE = re.compile(r"(?<![\w])([va])\[(\d+):(\d+)\]")
_ONE = re.compile(r"(?<![\w\[:])([va])(\d+)\b")


def _regs(tok):
    out = set()
    for m in _RANGE.finditer(tok):
        out |= {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    tok = _RANGE.sub("", tok)
    for m in _ONE.finditer(tok):
        out.add(f"{m.group(1)}{m.group(2)}")
    return out


def _operands(text):
    parts = text.split(None, 1)
    if len(parts) < 2:
        return parts[0], []
    body = re.split(r"\s(?:op_sel|op_sel_hi|dst_sel|dst_unused|src0_sel|src1_sel|clamp|"
                    r"offset|glc|slc|nt|sc0|sc1|cbsz|abid|blgp|neg_lo|neg_hi)\b", parts[1])[0]
    return parts[0], [o.strip() for o in re.split(r",(?![^\[]*\])", body)]


def kernels(asm_text):
    """{kernel symbol: [lines]} for every kernel body in a device assembly file."""
    out, cur = {}, None
    for ln in asm_text.splitlines():
        m = re.match(r"^(_Z\w+):", ln)
        if m:
            cur = m.group(1)
            out[cur] = []
            continue
        if cur is not None and re.match(r"^\s*\.Lfunc_end", ln):
            cur = None
            continue
        if cur is not None:
            out[cur].append(ln)
    return out


def check_kernel(name, lines, raw=12, war=4, asm_to_mfma=2):
    """Findings for one kernel's lines (see the module docstring)."""
    in_asm = False
    hist = []  # dicts: op, dst, src, asm, ws, text, settled (mfma dst regs already waited on)
    found = []
    for ln in lines:
        if "ASMSTART" in ln:
            in_asm = True
            continue
        if "ASMEND" in ln:
            in_asm = False
            continue
        text = ln.split(";")[0].strip()
        if not text or text.endswith(":") or text.startswith("."):
            continue
        op, ops = _operands(text)
        if op == "s_nop":
            hist.append(dict(op=op, dst=set(), src=set(), asm=in_asm, ws=int(ops[0], 0) + 1,
                             text=text))
            continue
        vector = op.startswith("v_") and not op.startswith(("v_readfirstlane", "v_readlane"))
        if vector:
            dst = _regs(ops[0]) if ops else set()
            src = set().union(*[_regs(o) for o in ops[1:]]) if len(ops) > 1 else set()
            if "UNUSED_PRESERVE" in text or op.startswith("v_fma_mix"):
                src |= dst  # preserves (reads) the other half of its destination
        else:
            dst, src = set(), set().union(*[_regs(o) for o in ops]) if ops else set()
        touched = src | dst
        if in_asm:
            ws = 0
            for h in reversed(hist):
                if ws >= max(raw, war, 1):
                    break
                if ws < 1 and TRANS.match(h["op"]) and h["dst"] & src:
                    found.append(Finding("trans->asm", name, ws, h["text"], text))
                if "mfma" in h["op"]:
                    live = h["dst"] - h["settled"]
                    if ws < raw and live & touched:
                        found.append(Finding("mfma->asm", name, ws, h["text"], text))
                    if ws < war and h["srcc"] & dst:
                        found.append(Finding("asm-srcc-war", name, ws, h["text"], text))
                ws += h["ws"]
        else:
            # a compiled instruction: the compiler waited for any MFMA result it touches
            for h in hist:
                if "mfma" in h["op"]:
                    h["settled"] |= h["dst"] & touched
            ws = 0
            for h in reversed(hist):
                if ws >= asm_to_mfma:
                    break
                if h["asm"] and h["dst"] & src:
                    if "mfma" in op:
                        found.append(Finding("asm->mfma", name, ws, h["text"], text))
                    elif vector and ws < 1 and ("dst_sel:WORD" in h["text"]
                                                or "dst_sel:BYTE" in h["text"]
                                                or "mixhi" in h["op"]):
                        found.append(Finding("asm-dstsel->valu", name, ws, h["text"], text))
                ws += h["ws"]
        rec = dict(op=op, dst=dst, src=src, asm=in_asm, ws=1, text=text, settled=set(),
                   srcc=set())
        if "mfma" in op and len(ops) >= 4:
            rec["srcc"] = _regs(ops[3])
        hist.append(rec)
        if len(hist) > 96:
            hist = hist[-96:]
    return found


def check_asm(asm_text):
    """All findings of every kernel in a device assembly file."""
    out = []
    for name, lines in kernels(asm_text).items():
        out += check_kernel(name, lines)
    return out
