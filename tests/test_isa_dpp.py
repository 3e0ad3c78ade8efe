"""Wait states around hand-written cross-lane instructions, checked on the
code the compiler actually emits (CPU only: hipcc cross-compiles gfx950).

A VALU instruction with a DPP source, and a v_permlane16/32_swap, needs two
wait states after any VALU write of a VGPR it reads. The compiler inserts these
for the instructions it generates itself, but it does not count the results of
inline assembly as VALU writes, so the asm blocks carry their own s_nop
padding. What the compiler places between them (spill reloads, copies, index
arithmetic) is outside their control; this test compiles every source that
uses such inline assembly and checks each DPP / permlane-swap instruction of
every kernel against the rule.
"""

import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "local-research-small-language-model_amd")
sys.path.insert(0, PKG)
from sparda import build as B  # noqa: E402

WAIT_STATES = 2


def _vgprs(tok: str):
    tok = tok.strip()
    m = re.fullmatch(r"v(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def _operands(ins: str):
    parts = ins.split(None, 1)
    if len(parts) < 2:
        return []
    return [o.strip().split()[0] for o in parts[1].split(",") if o.strip()]


def _valu_writes(ins: str):
    op = ins.split()[0]
    if not op.startswith("v_"):
        return set()                        # SALU, memory and LDS results are not VALU writes
    ops = _operands(ins)
    if not ops:
        return set()
    if "swap" in op:                        # v_swap_b32, v_permlane*_swap write both operands
        out = set()
        for o in ops[:2]:
            out |= _vgprs(o)
        return out
    return _vgprs(ops[0])


def dpp_hazards(asm_lines):
    """List of (writer, dpp) pairs closer than WAIT_STATES; a label reached
    before the wait states are accounted for counts as a hazard too (the
    predecessor on another path is unknown)."""
    ins = []
    for l in asm_lines:
        s = l.split(";")[0].strip()
        if not s or s.startswith("."):
            if s.endswith(":"):
                ins.append(s)               # local labels such as .LBB3_4:
            continue
        ins.append(s)
    bad = []
    for i, l in enumerate(ins):
        op0 = l.split()[0]
        if l.endswith(":") or ("_dpp" not in op0 and "permlane" not in op0):
            continue
        reads = set()
        for o in _operands(l)[:3]:          # vdst (read by fmac / swap), src0, src1
            reads |= _vgprs(o)
        ws = 0
        for p in reversed(ins[max(0, i - 8):i]):
            if ws >= WAIT_STATES:
                break
            if p.endswith(":"):
                bad.append(("label " + p, l))
                break
            op = p.split()[0]
            if op == "s_nop":
                ws += int(p.split()[1], 0) + 1
                continue
            if _valu_writes(p) & reads:
                bad.append((p, l))
                break
            ws += 1
    return bad


def kernels(asm_text: str):
    """{kernel symbol: instruction lines} for every kernel in a device .s file."""
    out, cur = {}, None
    for l in asm_text.splitlines():
        m = re.match(r"^(_Z\S+):", l)
        if m:
            cur = m.group(1)
            out[cur] = []
            continue
        if cur is not None:
            # a kernel may end in several s_endpgm (early exits): read to its end label
            if l.startswith(".Lfunc_end"):
                cur = None
                continue
            out[cur].append(l)
    return out


def test_checker_flags_a_planted_hazard():
    planted = [
        "v_mov_b32_e32 v5, 0",
        "v_fmac_f32_dpp v5, v1, v2 row_newbcast:0 row_mask:0xf bank_mask:0xf",
    ]
    assert len(dpp_hazards(planted)) == 1
    swap = ["v_max_f32_e32 v4, v4, v5", "v_permlane16_swap_b32_e32 v4, v6"]
    assert len(dpp_hazards(swap)) == 1
    assert dpp_hazards([swap[0], "s_nop 1", swap[1]]) == []
    padded = [planted[0], "s_nop 1", planted[1]]
    assert dpp_hazards(padded) == []
    one_short = [planted[0], "s_nop 0", planted[1]]
    assert len(dpp_hazards(one_short)) == 1
    spill = ["v_accvgpr_read_b32 v2, a7", "v_add_u32_e32 v9, v9, v8", planted[1]]
    assert len(dpp_hazards(spill)) == 1
    unrelated = ["v_mov_b32_e32 v7, 0", planted[1]]
    assert dpp_hazards(unrelated) == []
    after_label = [".LBB0_3:", planted[1]]
    assert len(dpp_hazards(after_label)) == 1


def _dpp_sources():
    """Sources whose kernels use DPP or permlane-swap inline assembly (also
    through the shared headers)."""
    hdr = {h: open(os.path.join(B.CSRC, h)).read() for h in os.listdir(B.CSRC) if h.endswith(".h")}
    asm_hdr = [h for h, t in hdr.items() if re.search(r"asm\s*\(.*(_dpp|permlane)", t)]
    out = []
    for src in B.sources():
        text = open(src).read()
        if re.search(r"asm\s*\(.*(_dpp|permlane)", text) or any(f'"{h}"' in text for h in asm_hdr):
            out.append(src)
    return out


@pytest.mark.skipif(shutil.which(B.HIPCC) is None and not os.path.exists(B.HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", [os.path.basename(s) for s in _dpp_sources()])
def test_emitted_dpp_wait_states(src, tmp_path):
    path = os.path.join(B.CSRC, src)
    out = tmp_path / (src + ".s")
    cmd = [B.HIPCC, *B.FLAGS, "--cuda-device-only", "-S", path, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    ks = kernels(out.read_text())
    n_dpp = 0
    problems = []
    for name, lines in ks.items():
        n_dpp += sum(1 for l in lines if "_dpp" in l.split(";")[0] or "permlane" in l.split(";")[0])
        for w, d in dpp_hazards(lines):
            problems.append(f"{name[:60]}: {w} -> {d}")
    assert n_dpp > 0, "no DPP / permlane-swap instructions found; the check would be vacuous"
    assert not problems, "\n".join(problems[:20])
