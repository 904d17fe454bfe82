"""The direct global->LDS copies are inline assembly (``common.h``: dma_buf16, dma_buf4, ...), and
the compiler inserts no wait states around inline assembly.  This CPU test compiles every source
that issues such copies to gfx950 assembly with the library's flags and checks the generated code
for the two GFX9 hazards that apply to them:

* an SGPR the copy reads (buffer descriptor, scalar offset) written by a VALU instruction
  (v_readfirstlane, v_readlane, a VALU carry-out) fewer than 5 wait states earlier: the copy would
  read a stale value (a build that spilled a copy's scalar offset through v_readlane failed the
  Polar parity test this way);
* m0 (the copy's LDS address) written fewer than 1 wait state before the copy.

Every copy is also checked to be one of the expected instructions, so a new copy form is noticed.
"""

import re
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from atma_amd import _build

SOURCES = ["polar_prefill.hip", "gated_delta_chunk16.hip", "polar_backward.hip", "gemm_gated.hip"]
COPIES = ("buffer_load_dwordx4", "buffer_load_dword", "global_load_lds_dwordx4")
# VALU instructions that write an SGPR: the destination, or the carry-out in the second slot
VALU_SGPR_FIRST = re.compile(r"^(v_readfirstlane_b32|v_readlane_b32|v_cmpx?_\w+_e64|v_div_scale_\w+)$")
VALU_SGPR_SECOND = re.compile(r"^(v_add_co_u32|v_sub_co_u32|v_subrev_co_u32|v_addc_co_u32|v_subb_co_u32|"
                              r"v_subbrev_co_u32|v_mad_u64_u32|v_mad_i64_i32)(_e64)?$")
SALU_NO_DST = ("s_waitcnt", "s_nop", "s_barrier", "s_cbranch", "s_branch", "s_cmp", "s_bitcmp", "s_setprio",
               "s_sleep", "s_endpgm", "s_sendmsg", "s_trap", "s_setreg", "s_dcache", "s_icache", "s_sethalt")


def _sgprs(tok):
    tok = tok.strip(",")
    if tok in ("m0", "M0"):
        return {"m0"}
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _writes(op, toks):
    """(SGPRs written, written by a VALU instruction) for one instruction."""
    if VALU_SGPR_FIRST.match(op) and toks:
        return _sgprs(toks[0]), True
    if VALU_SGPR_SECOND.match(op) and len(toks) > 1:
        return _sgprs(toks[1]), True
    if op.startswith("s_") and toks and not op.startswith(SALU_NO_DST):
        return _sgprs(toks[0]), False
    return set(), False


def check_assembly(text):
    """Hazards found in one assembly listing, as readable strings."""
    found, hist, in_asm, func, copies = [], [], False, "?", 0
    for line in text.split("\n"):
        s = line.strip()
        m = re.match(r"^(_Z\w+):", s)
        if m:
            func, hist = m.group(1), []
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        parts = s.split()
        op, toks = parts[0], [t.strip(",") for t in parts[1:]]
        if in_asm and (s.endswith(" lds") or op.startswith("global_load_lds")):
            copies += 1
            if op not in COPIES:
                found.append(f"{func}: unexpected copy form '{s}'")
            reads = {"m0"}
            for t in toks[1:]:
                reads |= _sgprs(t)
            waits = 0
            for hop, written, valu, nops in reversed(hist):
                if not reads or waits >= 5:
                    break
                hit = written & reads
                if hit:
                    if "m0" in hit and waits < 1:
                        found.append(f"{func}: '{s}' reads m0 written by '{hop}' with no wait state")
                    if valu and hit - {"m0"}:
                        found.append(f"{func}: '{s}' reads SGPR {sorted(hit - {'m0'})} written by '{hop}' "
                                     f"{waits} wait states earlier")
                    reads -= hit
                waits += nops
        written, valu = _writes(op, toks)
        nops = int(toks[0], 0) + 1 if op == "s_nop" else 1
        hist.append((op, written, valu, nops))
        del hist[:-16]
    return found, copies


def test_checker_finds_planted_hazards():
    """The checker itself, on listings with the two hazards planted (text only, nothing runs)."""
    bad_sgpr = """_Zk:
    v_readlane_b32 s0, v254, 5
    v_writelane_b32 v255, s25, 29
    ;;#ASMSTART
    s_nop 0
    buffer_load_dword v3, s[8:11], s0 offen lds
    ;;#ASMEND
"""
    bad_m0 = """_Zk:
    s_mov_b32 s4, s7
    s_mov_b32 m0, s6
    ;;#ASMSTART
    buffer_load_dwordx4 v3, s[8:11], s4 offen lds
    ;;#ASMEND
"""
    shadowed = """_Zk:
    v_mad_u64_u32 v[4:5], s[4:5], v1, s2, v[4:5]
    s_mul_i32 s4, s4, s25
    s_mov_b32 m0, s47
    ;;#ASMSTART
    s_nop 0
    buffer_load_dwordx4 v8, s[28:31], s4 offen lds
    ;;#ASMEND
"""
    found, n = check_assembly(bad_sgpr)
    assert n == 1 and len(found) == 1 and "SGPR [0]" in found[0]
    found, n = check_assembly(bad_m0)
    assert n == 1 and len(found) == 1 and "m0" in found[0]
    found, n = check_assembly(shadowed)
    assert n == 1 and found == []


def test_generated_copies_have_their_wait_states(tmp_path):
    hipcc = _build.hipcc()

    def compile_one(name):
        out = tmp_path / (Path(name).stem + ".s")
        cmd = [hipcc, *_build.COMMON_FLAGS, *_build.DEVICE_FLAGS, "--cuda-device-only", "-S",
               f"-I{_build.INCLUDE}", f"-I{_build.CSRC}", str(_build.CSRC / name), "-o", str(out)]
        proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        assert proc.returncode == 0, proc.stdout[-2000:]
        return name, out.read_text()

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        listings = list(ex.map(compile_one, SOURCES))
    total = 0
    for name, text in listings:
        found, copies = check_assembly(text)
        assert found == [], f"{name}:\n" + "\n".join(found[:20])
        total += copies
    assert total > 100  # the prefill, recurrence and backward kernels all copy through LDS
