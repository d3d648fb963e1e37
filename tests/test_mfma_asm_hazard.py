"""The sources built with -amdgpu-mfma-vgpr-form (shield-sisa_amd/build.py VGPR_FORM_SOURCES) keep MFMA accumulators
in ordinary VGPRs.  The compiler inserts the MFMA -> VALU wait states for its own instructions, but not for operands of
inline asm, so no inline-asm instruction may read a raw MFMA result.  The only VALU instructions this build writes as
inline asm are the DPP tap chains (v_*_dpp ... row_newbcast, strip.hip); this test disassembles the gfx950 code
objects of the locally built objects and checks, by a reaching-definition analysis over each kernel's control flow,
that no such instruction reads a VGPR that an MFMA write can reach."""
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LLVM = Path("/opt/rocm/llvm/bin")
OBJ = ROOT / "shield-sisa_amd" / "_obj"

BRANCH = re.compile(r"^s_(cbranch_\w+|branch|setpc_b64|swappc_b64)$")
REG = re.compile(r"\bv(\d+)\b|\bv\[(\d+):(\d+)\]")
WRITES_FIRST = re.compile(r"^(v_|ds_read|ds_load|global_load|buffer_load|flat_load|scratch_load)")


def vregs(text):
    out = set()
    for m in REG.finditer(text):
        if m.group(1) is not None:
            out.add(int(m.group(1)))
        else:
            out.update(range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def parse(disasm: str):
    """{function: [(address, mnemonic, operand text, branch target or None)]} from llvm-objdump -d output."""
    funcs, cur = {}, None
    for line in disasm.splitlines():
        m = re.match(r"^([0-9a-f]+) <(.+)>:$", line)
        if m:
            cur = []
            funcs[m.group(2)] = (int(m.group(1), 16), cur)
            continue
        if cur is None or not line.startswith("\t"):
            continue
        body, _, comment = line.strip().partition("//")
        parts = body.split(None, 1)
        if not parts:
            continue
        am = re.match(r"\s*([0-9A-Fa-f]+):", comment)
        addr = int(am.group(1), 16) if am else None
        tm = re.search(r"<[^>+]+\+0x([0-9a-f]+)>", comment)
        cur.append((addr, parts[0], parts[1] if len(parts) > 1 else "", int(tm.group(1), 16) if tm else None))
    return funcs


def writes(mn, ops):
    """The VGPRs an instruction writes and whether an MFMA writes them."""
    if not WRITES_FIRST.match(mn) or mn.startswith(("v_cmp", "v_readlane", "v_readfirstlane")):
        return set(), False
    return vregs(ops.split(",", 1)[0]), mn.startswith("v_mfma")


SREG = re.compile(r"^s\[(\d+):(\d+)\]$|^vcc$")


def sgpr_step(mn, ops, consts):
    """Constant propagation over the 64-bit scalar flags the compiler threads between conditional blocks
    (s_mov_b64 of -1 / 0, then vcc = exec & s / exec & ~s before s_cbranch_vcc[n]z).  consts maps 's[a:b]' / 'vcc'
    to -1, 0 or 'nz' (nonzero); anything else written by a scalar instruction becomes unknown."""
    args = [x.strip() for x in ops.split(",")]
    if not args or not args[0]:
        return
    dst = args[0]
    if mn == "s_mov_b64" and len(args) == 2 and args[1] in ("-1", "0"):
        consts[dst] = int(args[1])
        return
    if mn in ("s_and_b64", "s_andn2_b64") and len(args) == 3 and dst == "vcc" and args[1] == "exec":
        v = consts.get(args[2])
        if v is not None and v != "nz":
            keep = (v == -1) if mn == "s_and_b64" else (v == 0)
            consts["vcc"] = "nz" if keep else 0   # exec is nonzero in a running wave
            return
    if mn.startswith("s_") and (SREG.match(dst) or dst.startswith("s")):
        consts.pop(dst, None)
        if dst.startswith("s["):
            lo, hi = map(int, dst[2:-1].split(":"))
            for k in list(consts):
                if k.startswith("s[") and k != dst:
                    a0, a1 = map(int, k[2:-1].split(":"))
                    if a0 <= hi and lo <= a1:
                        consts.pop(k)
    if mn.startswith("v_cmp") and (dst == "vcc" or "vcc" in ops.split(",")[0]):
        consts.pop("vcc", None)


def mask(regs):
    m = 0
    for r in regs:
        m |= 1 << r
    return m


def hazards(funcs):
    """(checked asm reads, violations) over every function.  Reaching definitions on each function's control flow
    graph, kept apart per combination of the scalar flags the compiler threads between conditional blocks (so the
    branches those flags decide are followed one way only): a bit set per VGPR that an MFMA write can reach.  An asm
    DPP instruction may read a VGPR only when no MFMA write can reach it."""
    checked, bad = 0, []
    for name, (start, ins) in funcs.items():
        if not any("row_newbcast" in ops for _, _, ops, _ in ins):
            continue   # no inline-asm DPP instruction in this kernel
        addr_index = {a: i for i, (a, _, _, _) in enumerate(ins)}
        leaders = {0}
        for i, (_, mn, _, t) in enumerate(ins):
            if BRANCH.match(mn) or mn == "s_endpgm":
                leaders.add(i + 1)
                if t is not None and start + t in addr_index:
                    leaders.add(addr_index[start + t])
        starts = sorted(x for x in leaders if x < len(ins))
        bounds = list(zip(starts, starts[1:] + [len(ins)]))
        block_of = {b0: k for k, (b0, _) in enumerate(bounds)}
        # per instruction: (asm read mask, write mask, MFMA?, scalar?)
        pre = []
        for addr, mn, ops, _ in ins:
            rd = 0
            if "row_newbcast" in ops:
                dst, _, srcs = ops.partition(",")
                rd = mask(vregs(srcs) | (vregs(dst) if "fmac" in mn else set()))
                checked += bin(rd).count("1")
            regs, mfma = writes(mn, ops)
            pre.append((rd, mask(regs), mfma, mn.startswith("s_") or mn.startswith("v_cmp")))
        entry = [dict() for _ in bounds]   # per block: scalar-flag constants (frozenset) -> MFMA-reach mask
        entry[0][frozenset()] = 0
        work = [(0, frozenset())]
        flagged = set()
        while work:
            k, key = work.pop()
            m = entry[k][key]
            consts = dict(key)
            b0, b1 = bounds[k]
            for i in range(b0, b1):
                rd, wr, mfma, scalar = pre[i]
                if rd & m:
                    flagged.add(i)
                if wr:
                    m = (m | wr) if mfma else (m & ~wr)
                if scalar:
                    sgpr_step(ins[i][1], ins[i][2], consts)
            _, mn, _, t = ins[b1 - 1]
            taken = None   # None: either way
            if mn in ("s_cbranch_vccnz", "s_cbranch_vccz") and consts.get("vcc") is not None:
                nz = consts["vcc"] == "nz"
                taken = nz if mn == "s_cbranch_vccnz" else not nz
            out = []
            if t is not None and BRANCH.match(mn) and start + t in addr_index and taken is not False:
                out.append(block_of[addr_index[start + t]])
            if (mn != "s_endpgm" and not mn.startswith(("s_branch", "s_setpc")) and b1 < len(ins)
                    and not (taken is True and mn.startswith("s_cbranch"))):
                out.append(block_of[b1])
            nkey = frozenset(consts.items())
            for n in out:
                cur = entry[n].get(nkey)
                if cur is None or (cur | m) != cur:
                    entry[n][nkey] = m if cur is None else (cur | m)
                    work.append((n, nkey))
        for i in sorted(flagged):
            addr, mn, ops, _ = ins[i]
            bad.append(f"{name} @{addr:#x}: {mn} {ops} reads a VGPR that an MFMA write can reach")
    return checked, bad


def disassemble(obj: Path, tmp: Path) -> str:
    fat = tmp / (obj.name + ".fatbin")
    co = tmp / (obj.name + ".co")
    subprocess.run([str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", str(obj), str(tmp / "x.o")],
                   check=True, capture_output=True)
    subprocess.run([str(LLVM / "clang-offload-bundler"), "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={fat}", f"--output={co}", "--unbundle"], check=True, capture_output=True)
    return subprocess.run([str(LLVM / "llvm-objdump"), "-d", "--mcpu=gfx950", str(co)], check=True,
                          capture_output=True, text=True).stdout


def vgpr_form_sources():
    sys.path.insert(0, str(ROOT / "shield-sisa_amd"))
    import build
    return sorted(build.VGPR_FORM_SOURCES)


def test_checker_flags_a_planted_hazard():
    text = """0000000000001000 <k>:
\tv_mfma_f32_16x16x32_f16 v[4:7], v[8:11], v[12:15], v[4:7] // 000000001000: 0
\tv_fmac_f32_dpp v20, v1, v5 row_newbcast:1 row_mask:0xf bank_mask:0xf // 000000001008: 0
\tv_add_f32_e32 v5, 1.0, v5                                // 000000001010: 0
\tv_fmac_f32_dpp v21, v1, v5 row_newbcast:2 row_mask:0xf bank_mask:0xf // 000000001014: 0
"""
    checked, bad = hazards(parse(text))
    assert checked == 6 and len(bad) == 1 and "@0x1008" in bad[0]


def flag_threaded(op):
    """A conditional MFMA path that sets a scalar flag, and an asm read whose branch that flag decides (the shape the
    compiler gives the strip kernels' rows outside the map)."""
    return f"""0000000000001000 <k>:
\ts_and_b64 vcc, exec, s[2:3]                       // 000000001000: 0
\ts_mov_b64 s[28:29], -1                           // 000000001004: 0
\ts_cbranch_vccnz 3                                // 000000001008: 0 <k+0x18>
\tv_mfma_f32_16x16x32_f16 v[4:7], v[8:11], v[12:15], v[4:7] // 00000000100C: 0
\ts_mov_b64 s[28:29], 0                            // 000000001010: 0
\ts_nop 0                                          // 000000001014: 0
\t{op} vcc, exec, s[28:29]                         // 000000001018: 0
\ts_cbranch_vccnz 2                                // 00000000101C: 0 <k+0x28>
\tv_fmac_f32_dpp v20, v1, v5 row_newbcast:1 row_mask:0xf bank_mask:0xf // 000000001020: 0
\ts_endpgm                                         // 000000001024: 0
\tv_add_f32_e32 v5, 1.0, v5                        // 000000001028: 0
\tv_fmac_f32_dpp v21, v1, v5 row_newbcast:2 row_mask:0xf bank_mask:0xf // 00000000102C: 0
\ts_endpgm                                         // 000000001030: 0
"""


def test_checker_follows_flag_threaded_branches():
    # flag 0 (MFMA path) -> vcc = exec -> jump over the read: no MFMA write reaches it
    assert hazards(parse(flag_threaded("s_andn2_b64")))[1] == []
    # the same with the flag's sense inverted: the MFMA path falls through into the read
    bad = hazards(parse(flag_threaded("s_and_b64")))[1]
    assert len(bad) == 1 and "@0x1020" in bad[0]


@pytest.mark.parametrize("src", vgpr_form_sources())
def test_no_inline_asm_reads_an_mfma_result(src, tmp_path):
    obj = OBJ / (src + ".o")
    if not obj.exists() or not (LLVM / "clang-offload-bundler").exists():
        pytest.skip(f"{obj} not built (run __graft_entry__.build()) or no ROCm LLVM tools")
    funcs = parse(disassemble(obj, tmp_path))
    assert funcs, "no functions disassembled"
    checked, bad = hazards(funcs)
    assert not bad, "\n".join(bad[:20])
    if src == "strip.hip":
        assert checked > 10000, checked   # the DPP tap chains were found and checked
