"""gfx950 hazards that the compiler does not check inside inline assembly.

The HBM -> LDS copies (``global_load_lds_dwordx4``) are inline assembly
(``mlir-toy_amd/csrc/lds_dma.h``), so LLVM's hazard recognizer does not see
them, and the assembly itself must cover two hazards:

* a VALU write of an SGPR (``v_readfirstlane_b32`` of the copy's base) read
  by a VMEM instruction needs 5 wait states;
* an SALU write of M0 read by an LDS DMA needs 1 wait state.

Each wait state is one issued instruction (``s_nop N`` gives N + 1). This
test compiles every kernel source to gfx950 assembly with the build's own
flags. For every copy it then walks back over the instructions that precede
it in program order. It pins a paged-decode bug in which a base looked up
in the block table was written by ``v_readfirstlane`` two instructions
before the copy that read it. The copy saw the previous base and loaded
another step's tokens, with no fault.

The fp8 decode's K-code register loads are inline assembly as well: the
compiled code is checked for the order its waits rely on (each step's four K
loads followed by its four V copies, and every wait before a K buffer is read
leaving only the step's V copies and whole later steps in flight).

The same compiled code also holds the kernels to the register budgets their
speed depends on (test_kernel_register_budgets): the selective scan's
output kernel within 96 VGPRs (five waves per SIMD), the production prefill
within 256 (two per SIMD), and these and the decode kernels without scratch.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "mlir-toy_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
SOURCES = sorted(CSRC.glob("*.hip"))

VALU_SGPR_TO_VMEM = 5
M0_TO_LDS_DMA = 1


def _build_flags() -> list[str]:
    """HIPFLAGS of the library's Makefile (continuation lines joined)."""
    text = (CSRC / "Makefile").read_text().replace("\\\n", " ")
    m = re.search(r"^HIPFLAGS\s*\?=\s*(.+)$", text, re.M)
    assert m, "HIPFLAGS not found in the Makefile"
    return m.group(1).split()


def _sgprs(tok: str) -> set[int]:
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _instructions(asm: str) -> list[tuple[str, list[str]]]:
    out = []
    for line in asm.splitlines():
        if not line.startswith("\t") or line.lstrip().startswith((".", ";")):
            continue
        body = line.split(";", 1)[0].strip()
        if not body:
            continue
        mnem, _, rest = body.partition(" ")
        # operands without trailing modifiers ("s[36:37] nt" -> "s[36:37]")
        ops = [o.split()[0] for o in rest.split(",") if o.strip()] if rest else []
        out.append((mnem, ops))
    return out


def _valu_sgpr_dests(mnem: str, ops: list[str]) -> set[int]:
    """SGPRs a VALU instruction writes: the scalar destination of readlane /
    readfirstlane / compares, and the carry-out of *_co_* and div_scale forms."""
    if not mnem.startswith("v_") or not ops:
        return set()
    dests = _sgprs(ops[0])
    if len(ops) > 1 and ("_co_" in mnem or mnem.startswith(("v_addc", "v_subb", "v_div_scale"))):
        dests |= _sgprs(ops[1])
    return dests


def hazards(asm: str) -> list[str]:
    """Copies whose SGPR base or M0 is written too few wait states before."""
    ins = _instructions(asm)
    found = []
    for j, (mnem, ops) in enumerate(ins):
        # the LDS copies (vaddr, saddr) and the register loads of the fp8 K
        # codes (vdst, vaddr, saddr), both inline assembly
        # (only the LDS copies read M0)
        reads_m0 = mnem.startswith("global_load_lds")
        if reads_m0:
            base = _sgprs(ops[1]) if len(ops) > 1 else set()
        elif mnem == "global_load_dwordx4" and len(ops) > 2:
            base = _sgprs(ops[2])
        else:
            continue
        waits = 0
        for k in range(j - 1, -1, -1):
            pm, pops = ins[k]
            if pm == "s_nop":
                waits += int(pops[0], 0) + 1
                continue
            if base and waits < VALU_SGPR_TO_VMEM and _valu_sgpr_dests(pm, pops) & base:
                found.append(f"copy #{j} ({' '.join([mnem] + ops)}): base written by "
                             f"{pm} {', '.join(pops)} {waits} wait states before")
                break
            if (reads_m0 and pm.startswith("s_") and pops and pops[0] == "m0"
                    and waits < M0_TO_LDS_DMA):
                found.append(f"copy #{j}: M0 written by {pm} {waits} wait states before")
                break
            waits += 1
            if waits >= VALU_SGPR_TO_VMEM:
                break
    return found


KLOAD = re.compile(r"^[ \t]*global_load_dwordx4 (v\[\d+:\d+\]), [^;\n]* nt[ \t]*$", re.M)
KWAIT = re.compile(r";\s*kload_wait (v\[\d+:\d+\]) (v\[\d+:\d+\]) (v\[\d+:\d+\]) "
                   r"(v\[\d+:\d+\])")


def kload_findings(asm: str) -> tuple[int, list[str]]:
    """The fp8 decode loads K codes into registers by inline assembly and
    marks each wait for them with a "; kload_wait" comment naming the
    registers its statement ties. Per kernel: every register quad a wait
    names must be the destination of one of the kernel's K loads (a copy made
    before the wait would name other registers and read data still in
    flight), and the kernel must not spill (a spill store would read it
    too). Returns (number of waits, findings)."""
    found, waits = [], 0
    for name, body in re.findall(r"^(\S+):\s*;\s*@\S+\n(.*?)^\.Lfunc_end", asm, re.S | re.M):
        dests = set(KLOAD.findall(body))
        named = [q for m in KWAIT.findall(body) for q in m]
        if not named:
            continue
        waits += len(named) // 4
        for q in named:
            if q not in dests:
                found.append(f"{name}: kload_wait names {q}, which no K load writes")
        if re.search(r"^\s*(scratch_|buffer_store)", body, re.M):
            found.append(f"{name}: spills while K loads are in flight")
    return waits, found


VMEM = ("global_", "buffer_", "flat_", "scratch_")
R8P = 4  # decode_partial_ring8: 32-token steps in flight (K buffers, V ring slots)


def kload_order_findings(asm: str, in_flight: int = R8P) -> list[str]:
    """The order the fp8 decode's waits rely on, per kernel with K-load waits.

    * Issue: each step is four K loads followed at once by the four LDS copies
      of its V tile, so 4 + 8 l vector-memory operations are issued after a
      K buffer's last load when l later steps follow it.
    * Wait: each s_waitcnt vmcnt(N) between a kload_wait and the vector-memory
      operation before it is one of the kernel's per-`later` choices,
      N = 4 + 8 l with 0 <= l < in_flight (the step's own V copies plus l
      later steps may stay in flight), and each of those in_flight choices
      occurs. That a wait never exceeds the operations actually issued after
      the buffer then rests on l counting the later steps issued (the
      kernel's `later`), which every ragged-length parity case exercises.
    Operations of other kinds issued in between only make a wait retire the
    K loads earlier. Returns the findings."""
    found = []
    allowed = {4 + 8 * l for l in range(in_flight)}
    for name, body in re.findall(r"^(\S+):\s*;\s*@\S+\n(.*?)^\.Lfunc_end", asm, re.S | re.M):
        if "kload_wait" not in body:
            continue
        seq = []  # ("K" | "C" | "M" other memory | "W" | "N" wait, vmcnt)
        for line in body.splitlines():
            t = line.strip()
            if t.startswith(VMEM):
                m = t.split()[0]
                if KLOAD.match(line):
                    seq.append(("K", None))
                else:
                    seq.append(("C" if m.startswith("global_load_lds") else "M", None))
            elif "kload_wait" in t:
                seq.append(("W", None))
            elif t.startswith("s_waitcnt") and "vmcnt(" in t:
                seq.append(("N", int(re.search(r"vmcnt\((\d+)\)", t).group(1))))
        mem = [k for k, _ in seq if k in "KCM"]
        i = 0
        while i < len(mem):
            if mem[i] != "K":
                i += 1
                continue
            j = i
            while j < len(mem) and mem[j] == "K":
                j += 1
            c = j
            while c < len(mem) and mem[c] == "C":
                c += 1
            if j - i != 4 or c - j != 4:
                found.append(f"{name}: a step issues {j - i} K loads then {c - j} LDS copies "
                             f"(want 4 and 4)")
            i = c
        seen = set()
        for w, (kind, _) in enumerate(seq):
            if kind != "W":
                continue
            k = w - 1
            while k >= 0 and seq[k][0] == "N":
                n = seq[k][1]
                seen.add(n)
                if n not in allowed:
                    found.append(f"{name}: vmcnt({n}) before a kload_wait is not one of "
                                 f"{sorted(allowed)}")
                k -= 1
            if k == w - 1:
                found.append(f"{name}: a kload_wait with no vmcnt wait after the last load")
        if seen != allowed:
            found.append(f"{name}: waits before kload_wait {sorted(seen)}, want {sorted(allowed)}")
    return found


def test_kload_order_checker():
    step = ("\tglobal_load_dwordx4 v[18:21], v140, s[20:21] nt\n" * 4
            + "\tglobal_load_lds_dwordx4 v61, s[36:37] nt\n" * 4)
    waits = "".join(f"\ts_waitcnt vmcnt({n})\n" for n in (28, 20, 12, 4))
    good = ("k:  ; @k\n" + step * 4 + waits
            + "\t; kload_wait v[18:21] v[22:25] v[26:29] v[30:33]\n.Lfunc_end0:\n")
    assert kload_order_findings(good) == []
    assert len(kload_order_findings(good.replace("vmcnt(12)", "vmcnt(13)"))) == 2
    assert kload_order_findings(good.replace("vmcnt(28)", "vmcnt(36)"))
    short = good.replace(step, step.replace("\tglobal_load_lds_dwordx4 v61, s[36:37] nt\n", "", 1), 1)
    assert kload_order_findings(short)
    late = good.replace(step, step.replace("nt\n\tglobal_load_lds", "nt\n\tglobal_load_dword v1, "
                                           "v[2:3], off\n\tglobal_load_lds", 1), 1)
    assert kload_order_findings(late)


def test_kload_checker_flags_a_copy():
    ok = ("k:  ; @k\n\tglobal_load_dwordx4 v[18:21], v140, s[20:21] nt\n"
          "\t; kload_wait v[18:21] v[22:25] v[26:29] v[30:33]\n.Lfunc_end0:\n")
    loads = "".join(f"\tglobal_load_dwordx4 v[{a}:{a + 3}], v140, s[20:21] nt\n"
                    for a in (22, 26, 30))
    good = ok.replace("\t; kload", loads + "\t; kload")
    assert kload_findings(good) == (1, [])
    copied = good.replace("kload_wait v[18:21]", "kload_wait v[40:43]")
    assert len(kload_findings(copied)[1]) == 1
    spilled = good.replace("\t; kload", "\tscratch_store_dwordx4 off, v[18:21], s33\n\t; kload")
    assert len(kload_findings(spilled)[1]) == 1


def test_checker_flags_a_stale_base():
    """The checker itself: a base written by v_readfirstlane one instruction
    before the copy is flagged; with s_nop 4 in between it is not."""
    bad = ("\tv_readfirstlane_b32 s37, v15\n\tv_readfirstlane_b32 s36, v14\n"
           "\ts_nop 0\n\tglobal_load_lds_dwordx4 v61, s[36:37] nt\n")
    good = bad.replace("s_nop 0", "s_nop 4")
    m0 = "\ts_mov_b32 m0, s4\n\tglobal_load_lds_dwordx4 v1, off\n"
    assert len(hazards(bad)) == 1
    assert hazards(good) == []
    assert len(hazards(m0)) == 1 and hazards(m0.replace("\tglobal", "\ts_nop 0\n\tglobal")) == []
    # a register load does not read M0
    assert hazards("\ts_mov_b32 m0, s4\n\tglobal_load_dwordx4 v[4:7], v[2:3], off\n") == []


@pytest.fixture(scope="module")
def compiled(tmp_path_factory):
    """Every kernel source compiled to gfx950 assembly with the build's flags
    (file name -> assembly text)."""
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    tmp = tmp_path_factory.mktemp("isa")
    flags = _build_flags()
    procs = {}
    for src in SOURCES:
        out = tmp / (src.stem + ".s")
        procs[src.name] = (out, subprocess.Popen(
            [HIPCC, *flags, "--cuda-device-only", "-S", "-o", str(out), str(src)],
            stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, text=True))
    asm = {}
    for name, (out, p) in procs.items():
        _, err = p.communicate(timeout=600)
        assert p.returncode == 0, f"{name}: {err[-2000:]}"
        asm[name] = out.read_text()
    return asm


def test_lds_dma_wait_states(compiled):
    report, copies, kwaits = [], 0, 0
    for name, asm in compiled.items():
        copies += asm.count("global_load_lds_dwordx4")
        report += [f"{name}: {h}" for h in hazards(asm)]
        n, found = kload_findings(asm)
        kwaits += n
        report += [f"{name}: {f}" for f in found]
        report += [f"{name}: {f}" for f in kload_order_findings(asm)]
    assert copies > 0, "no LDS DMA copies found: the checker is looking at the wrong code"
    assert kwaits > 0, "no K-load waits found: the checker is looking at the wrong code"
    assert not report, "\n".join(report)


def kernel_resources(asm: str) -> dict[str, tuple[int, int]]:
    """Kernel symbol -> (VGPRs, AGPRs included, and scratch bytes per lane)
    from the code object's kernel descriptors."""
    out = {}
    for m in re.finditer(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", asm, re.S):
        body = m.group(2)
        vgpr = int(re.search(r"\.amdhsa_next_free_vgpr (\d+)", body).group(1))
        scratch = int(re.search(r"\.amdhsa_private_segment_fixed_size (\d+)", body).group(1))
        out[m.group(1)] = (vgpr, scratch)
    return out


# Register budgets the performance depends on: (symbol pattern, VGPR limit,
# why). Every kernel listed must also run without scratch.
BUDGETS = [
    # the selective scan's output kernel: five resident work-groups per CU
    # (five waves per SIMD) is what config 4's 1280 work-groups need
    (r"selective_scan_out", 96, "five waves per SIMD"),
    # the production prefill (two LDS stages): two work-groups per CU
    (r"attn_fwd_d128INS_7Bf16TagELb1ELi2ELb0E", 256, "two waves per SIMD"),
    # the decode partial kernels: a scratch reload's wait would retire the
    # copies in flight
    (r"decode_partial_ring", 512, "no scratch"),
]


def test_kernel_register_budgets(compiled):
    res = {}
    for asm in compiled.values():
        res.update(kernel_resources(asm))
    report = []
    for pat, limit, why in BUDGETS:
        hits = {k: v for k, v in res.items() if re.search(pat, k)}
        assert hits, f"no kernel matches {pat}: the check is looking at the wrong code"
        for k, (vgpr, scratch) in hits.items():
            if vgpr > limit or scratch:
                report.append(f"{k}: {vgpr} VGPRs (limit {limit}, {why}), {scratch} B scratch")
    assert not report, "\n".join(report)


def test_kernel_resources_parser():
    asm = ("\t.amdhsa_kernel _Zfoo\n\t\t.amdhsa_private_segment_fixed_size 8\n"
           "\t\t.amdhsa_next_free_vgpr 97\n\t.end_amdhsa_kernel\n")
    assert kernel_resources(asm) == {"_Zfoo": (97, 8)}
