"""Checks on the gfx950 code the library was built into (our own build, disassembled with ROCm's llvm-objdump): the
kernels that stream K slices into LDS with direct-to-LDS loads wait for them with `s_waitcnt vmcnt(N)`, N > 0, so
that later loads may stay in flight.  That is only correct while the instruction order the counts assume holds:

* w4_big_kernel (prefill, two register sets): the N loads after the last x load of a slice are the next weight
  fetch, so at least N vector-memory loads must follow the last `global_load_lds` before each such wait;
* mm_ring_kernel (W8A8 small M, S-stage ring): each loop iteration issues exactly the NI direct-to-LDS loads of one
  slice and no other vector-memory load, and waits with vmcnt((S - 2) * NI) ("slice kt + 1 has landed");
* w4_ring_kernel (W4 on the CDNA4 layout, 33..64 rows or long K): the same rule with NI = 4 MB / BW + T + 2 buffer
  loads into LDS per step;
* w8a16_ring_kernel (W8A16, 3..64 rows): the same rule with NI = 4 MB / BW + 2 T + 1 (two loads per weight tile, no
  zero-points);
* w4_pp_kernel (W4A16 / W8A16 ping-pong prefill): every wavefront issues 4 x loads and 3 staging loads per V phase
  (10 / 14 before its first wait), and waits only with vmcnt(7) (a staging group with an x and a staging group after
  it) or vmcnt(10) (an x group with three groups after it); between two waits it issues one V phase's 7 loads or none.

A compiler that reorders, splits or adds a load there breaks the check here, on the CPU, instead of silently racing on
the GPU.  No GPU is used."""
from __future__ import annotations

import os
import re
import shutil
import struct
import subprocess
import tempfile

import pytest

from forge_amd import _lib

OBJDUMP = next((p for p in ("/opt/rocm/llvm/bin/llvm-objdump", shutil.which("llvm-objdump") or "") if p and
                os.path.exists(p)), None)
pytestmark = pytest.mark.skipif(OBJDUMP is None or not os.path.exists(_lib.LIB_PATH),
                                reason="needs the built library and ROCm's llvm-objdump")
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _section(path: str, name: str) -> bytes:
    """Bytes of an ELF64 little-endian section by name."""
    data = open(path, "rb").read()
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", data, 0x3A)
    headers = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    strtab = headers[shstrndx]
    names = data[strtab[4]:strtab[4] + strtab[5]]
    for h in headers:
        if names[h[0]:names.index(b"\0", h[0])].decode() == name:
            return data[h[4]:h[4] + h[5]]
    raise AssertionError(f"{name} not in {path}")


def _gfx950_objects(fatbin: bytes) -> list[bytes]:
    """The gfx950 code objects of the concatenated offload bundles (one per compiled source file)."""
    out, pos = [], fatbin.find(BUNDLE_MAGIC)
    while pos != -1:
        n, = struct.unpack_from("<Q", fatbin, pos + 24)
        p = pos + 32
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            triple = fatbin[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if "gfx950" in triple:
                out.append(fatbin[pos + off:pos + off + size])
        pos = fatbin.find(BUNDLE_MAGIC, pos + 1)
    return out


INSN = re.compile(r"^\s+([a-z0-9_]+)\s*(.*?)\s*//\s*([0-9A-F]+):(.*)$")
FUNC = re.compile(r"^[0-9a-f]+ <(\S+)>:")


@pytest.fixture(scope="module")
def kernels() -> dict[str, list[tuple[int, str, str]]]:
    """function name -> [(address, mnemonic, operands)] for every kernel of the library."""
    funcs: dict[str, list[tuple[int, str, str]]] = {}
    with tempfile.TemporaryDirectory() as tmp:
        for i, co in enumerate(_gfx950_objects(_section(_lib.LIB_PATH, ".hip_fatbin"))):
            path = os.path.join(tmp, f"c{i}.co")
            with open(path, "wb") as f:
                f.write(co)
            text = subprocess.run([OBJDUMP, "-d", "--no-show-raw-insn", path], capture_output=True, text=True,
                                  check=True).stdout
            cur = None
            for line in text.splitlines():
                m = FUNC.match(line)
                if m:
                    cur = funcs.setdefault(m.group(1), [])
                    continue
                m = INSN.match(line)
                if m and cur is not None:
                    cur.append((int(m.group(3), 16), m.group(1), m.group(2) + " " + m.group(4)))
    return funcs


def _vmem(mnem: str) -> bool:
    return mnem.startswith(("global_load", "buffer_load"))


def _lds_dma(mnem: str, ops: str = "") -> bool:
    """A direct-to-LDS load: global_load_lds_* or a buffer load with the lds modifier."""
    return _vmem(mnem) and ("_lds" in mnem or re.search(r"\blds\b", ops.split("//")[0]) is not None)


def _vmcnt(mnem: str, ops: str) -> int | None:
    m = re.search(r"vmcnt\((\d+)\)", ops) if mnem == "s_waitcnt" else None
    return int(m.group(1)) if m else None


def _barrier_waits(code: list[tuple[int, str, str]]) -> list[tuple[int, int]]:
    """(index, N) of each `s_waitcnt vmcnt(N)`, N > 0, right before an `s_barrier`: the kernels' own waits that
    publish a slice in LDS to the workgroup (the compiler's waits for register loads are its own business)."""
    return [(i, n) for i, (_, m, o) in enumerate(code[:-1])
            if (n := _vmcnt(m, o)) and code[i + 1][1] == "s_barrier"]


def _dma_landed(code: list[tuple[int, str, str]], idx: int) -> bool:
    """Whether every direct-to-LDS load before code[idx] has landed once code[idx] (a vmcnt wait) retires."""
    last_dma = max((i for i in range(idx) if _lds_dma(code[i][1], code[i][2])), default=None)
    if last_dma is None:
        return True
    # vmcnt(k) leaves only the k most recent loads in flight: the direct-to-LDS load has landed once some wait from it
    # to here allows no more than the loads issued after it
    younger = 0
    for _, m2, o2 in code[last_dma + 1:idx + 1]:
        k = _vmcnt(m2, o2)
        if k is not None and younger >= k:
            return True
        younger += _vmem(m2)
    return False


def test_the_check_catches_a_reordered_load():
    """The rule on hand-made sequences: three weight loads after the x rows satisfy vmcnt(3); one moved above the
    x rows does not, unless a full wait already drained everything."""
    dma, ld, bar = (0, "global_load_lds_dwordx4", ""), (0, "global_load_dwordx4", ""), (0, "s_barrier", "")
    wait = lambda n: (0, "s_waitcnt", f"vmcnt({n}) lgkmcnt(0)")  # noqa: E731
    assert _dma_landed([dma, dma, ld, ld, ld, wait(3), bar], 5)
    assert not _dma_landed([ld, dma, dma, ld, ld, wait(3), bar], 5)
    assert _dma_landed([ld, dma, dma, ld, wait(0), ld, wait(3), bar], 6)


def test_prefill_waits_leave_only_the_weight_fetch_in_flight(kernels):
    found = 0
    for name, code in kernels.items():
        if "w4_big_kernel" not in name or not name.endswith("iiiii") or "Li2EEEv" not in name:
            continue
        for idx, n in _barrier_waits(code):
            assert any(_lds_dma(m, o) for _, m, o in code[:idx]), name
            assert _dma_landed(code, idx), f"{name}: the vmcnt({n}) at {idx} leaves a direct-to-LDS load in flight"
            found += 1
    assert found >= 16, f"expected the two-register-set prefill instances, checked {found} waits"


def _successors(code: list[tuple[int, str, str]], addr: dict[int, int], i: int) -> list[int]:
    """Indices control can reach from code[i] (branch targets resolved from the disassembler's <func+0xoff>)."""
    mnem, ops = code[i][1], code[i][2]
    if mnem == "s_endpgm":
        return []
    nxt = [i + 1] if i + 1 < len(code) else []
    if mnem.startswith(("s_cbranch", "s_branch")):
        tgt = re.search(r"<\S+\+0x([0-9a-f]+)>", ops)
        t = [addr[code[0][0] + int(tgt.group(1), 16)]] if tgt else []
        return t if mnem.startswith("s_branch") else nxt + t
    return nxt


def _check_ring_loops(name: str, code: list[tuple[int, str, str]], ni: int, s: int) -> int:
    """Every barrier wait of a ring kernel is vmcnt((S - 2) * NI); every path from kernel entry to the first wait issues
    (S - 1) * NI direct-to-LDS loads, and every path from one wait to the next exactly NI (one step's; however the
    compiler lays out or unrolls the loop) and no other vector-memory load, so each wait leaves exactly the S - 2
    younger steps in flight; a path from the last wait to the end issues one step's loads or none.  Returns the waits
    checked."""
    addr = {a: i for i, (a, _, _) in enumerate(code)}
    waits = _barrier_waits(code)
    assert waits and all(n == (s - 2) * ni for _, n in waits), (name, waits, ni, s)
    wset = {w for w, _ in waits}

    def walk(starts: list[int]) -> set[tuple[str, int, int]]:
        """(end kind, DMA count, any other load) over every path from code[k], k in starts, to the next wait or the
        end."""
        ends, seen, todo = set(), set(), [(k, 0, 0) for k in starts]
        while todo:
            i, dma, other = todo.pop()
            if (i, dma, other) in seen:
                continue
            seen.add((i, dma, other))
            assert dma <= s * ni and len(seen) < 200000, f"{name}: a path from {starts} issues {dma} DMA loads"
            if i in wset:
                ends.add(("wait", dma, other))
                continue
            m, o = code[i][1], code[i][2]
            dma2, other2 = dma + _lds_dma(m, o), min(1, other + (_vmem(m) and not _lds_dma(m, o)))
            succ = _successors(code, addr, i)
            if not succ:
                ends.add(("end", dma2, other2))
            todo.extend((k, dma2, other2) for k in succ)
        return ends

    first = walk([0])
    assert {(k, d) for k, d, _ in first if k == "wait"} == {("wait", (s - 1) * ni)}, (name, first)
    for w, _ in waits:
        for kind, dma, other in walk(_successors(code, addr, w)):
            assert dma == ni or (kind == "end" and dma == 0), \
                f"{name}: a path from the wait at {w} to the next {kind} issues {dma} DMA loads"
            assert kind == "end" or other == 0, f"{name}: a step issues {other} other loads"
    return len(waits)


def test_ring_step_check_rejects_a_planted_extra_load():
    """The path walk on a hand-written two-stage loop (NI = 2, S = 3): accepted as written, rejected when one step
    issues a third direct-to-LDS load or a register load, or when the wait count is off by one."""
    def prog(extra: str = "", wait: int = 2) -> list[tuple[int, str, str]]:
        body = [("buffer_load_dword", "v0, v1, s[0:3], 0 offen lds"), ("buffer_load_dword", "v0, v1, s[0:3], 0 offen lds")]
        loop = [("s_waitcnt", f"vmcnt({wait}) lgkmcnt(0)"), ("s_barrier", "")] + body
        if extra:
            loop.append(("buffer_load_dword", extra))
        loop += [("v_mfma_f32_16x16x32_bf16", "v[0:3], v[4:7], v[8:11], v[0:3]"), ("s_cbranch_scc1", "<k+0x{:x}>")]
        code = body * 2 + loop + [("s_endpgm", "")]
        out = []
        for i, (m, o) in enumerate(code):
            out.append((0x1000 + 4 * i, m, o.format(4 * 4) if m == "s_cbranch_scc1" else o))
        return out

    assert _check_ring_loops("ok", prog(), 2, 3) == 1
    for bad in (prog("v0, v1, s[0:3], 0 offen lds"), prog("v2, v1, s[0:3], 0 offen"), prog(wait=3)):
        with pytest.raises(AssertionError):
            _check_ring_loops("bad", bad, 2, 3)


def test_ring_kernel_loop_issues_one_slice_and_waits_for_the_next(kernels):
    found = 0
    for name, code in kernels.items():
        if "mm_ring_kernel" not in name:
            continue
        bm, bn, wm, wn, s = (int(v) for v in re.findall(r"Li(\d+)E", name)[:5])
        found += _check_ring_loops(name, code, (bm + bn) * 128 // 16 // (wm * wn * 64), s)
    assert found >= 4, f"expected the ring instances' loops, checked {found}"


def test_w4_ring_kernel_loop_issues_one_step_and_waits_for_the_next(kernels):
    found = 0
    for name, code in kernels.items():
        if "w4_ring_kernel" not in name:
            continue
        mb, t, bw, s = (int(v) for v in re.findall(r"Li(\d+)E", name)[:4])
        found += _check_ring_loops(name, code, 4 * mb // bw + t + 2, s)
    assert found >= 16, f"expected the W4 ring instances' loops, checked {found}"


def test_w8a16_ring_kernel_loop_issues_one_step_and_waits_for_the_next(kernels):
    found = 0
    for name, code in kernels.items():
        if "w8a16_ring_kernel" not in name:
            continue
        mb, t, bw, s = (int(v) for v in re.findall(r"Li(\d+)E", name)[:4])
        found += _check_ring_loops(name, code, 4 * mb // bw + 2 * t + 1, s)
    assert found >= 16, f"expected the W8A16 ring instances' loops, checked {found}"


def _check_pp(name: str, code: list[tuple[int, str, str]]) -> int:
    """The ping-pong kernel's load accounting: waits are vmcnt(7) or vmcnt(10); every path from entry issues 10 (team
    A: stg, x, stg) or 14 (team B: x, stg, x, stg) direct-to-LDS loads before the first wait; every path from a wait to
    the next issues 0 or 7 and no other vector-memory load.  The kernel branches on the wave-uniform team index with
    every lane active, so the exec-is-zero skips the compiler leaves around that if / else never fire: their taken
    edges are not walked.  Returns the waits checked."""
    addr = {a: i for i, (a, _, _) in enumerate(code)}

    def succ_of(i: int) -> list[int]:
        nxt = _successors(code, addr, i)
        return nxt[:1] if code[i][1] == "s_cbranch_execz" else nxt
    # the kernel's own waits; after the last barrier (the drain) the epilogue's waits for its register loads follow
    last_barrier = max(i for i, (_, m, _) in enumerate(code) if m == "s_barrier")
    waits = [(i, n) for i, (_, m, o) in enumerate(code[:last_barrier]) if (n := _vmcnt(m, o))]
    assert waits and all(n in (7, 10) for _, n in waits), (name, waits)
    wset = {w for w, _ in waits}

    def walk(starts: list[int]) -> set[tuple[str, int, int]]:
        ends, seen, todo = set(), set(), [(k, 0, 0) for k in starts]
        while todo:
            i, dma, other = todo.pop()
            if (i, dma, other) in seen:
                continue
            seen.add((i, dma, other))
            assert dma <= 14 and len(seen) < 400000, f"{name}: a path from {starts} issues {dma} DMA loads"
            if i in wset:
                ends.add(("wait", dma, other))
                continue
            m, o = code[i][1], code[i][2]
            dma2, other2 = dma + _lds_dma(m, o), min(1, other + (_vmem(m) and not _lds_dma(m, o)))
            succ = succ_of(i)
            if not succ:
                ends.add(("end", dma2, other2))
            todo.extend((k, dma2, other2) for k in succ)
        return ends

    first = {d for k, d, _ in walk([0]) if k == "wait"}
    assert first == {10, 14}, (name, first)
    for w, _ in waits:
        for kind, dma, other in walk(succ_of(w)):
            if kind == "wait":
                assert dma in (0, 7) and other == 0, f"{name}: {dma} DMA / {other} other loads between waits at {w}"
            else:
                assert dma == 0, f"{name}: a path from the wait at {w} to the end issues {dma} DMA loads"
    return len(waits)


def test_pp_kernel_issues_one_v_phase_between_waits(kernels):
    found = 0
    for name, code in kernels.items():
        if "w4_pp_kernel" in name:
            found += _check_pp(name, code)
    assert found >= 4 * 4, f"expected the four ping-pong instances' waits, checked {found}"


def test_pp_check_rejects_a_planted_extra_load():
    """The ping-pong walk on a hand-written team-B-like program (14 loads, wait, then a loop of 7 loads and a wait):
    accepted as written, rejected with an eighth load in the loop, a register load there, or a wait of 8."""
    def prog(extra: str = "", wait: int = 7, first: int = 10) -> list[tuple[int, str, str]]:
        dma = ("buffer_load_dwordx4", "v0, s[0:3], 0 offen lds")
        pro = [dma] * 14 + [("s_waitcnt", f"vmcnt({wait})"), ("s_barrier", "")]
        loop = [dma] * 7 + ([("buffer_load_dword", extra)] if extra else []) + \
            [("s_barrier", ""), ("s_waitcnt", f"vmcnt({wait})"), ("s_barrier", ""), ("s_cbranch_scc1", "<k+0x{:x}>")]
        team_a = [dma] * first + [("s_waitcnt", "vmcnt(7)"), ("s_barrier", "")]
        code = [("s_cbranch_scc0", "<k+0x{:x}>")] + pro + loop + [("s_branch", "<k+0x{:x}>")] + team_a + \
            [("s_waitcnt", "vmcnt(0)"), ("s_barrier", ""), ("s_endpgm", "")]
        loop0, a0 = 1 + len(pro), 1 + len(pro) + len(loop) + 1
        end = a0 + len(team_a)
        targets = {0: a0, loop0 + len(loop) - 1: loop0, a0 - 1: end}
        return [(0x1000 + 4 * i, m, o.format(4 * targets[i]) if i in targets else o) for i, (m, o) in enumerate(code)]

    assert _check_pp("ok", prog()) == 3
    for bad in (prog("v0, s[0:3], 0 offen lds"), prog("v2, s[0:3], 0 offen"), prog(wait=8), prog(first=11)):
        with pytest.raises(AssertionError):
            _check_pp("bad", bad)


VREG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
MFMA_AB_WAIT = 2  # wait states between a VALU write of a VGPR and an MFMA reading it as SrcA / SrcB


def _vgprs(text: str) -> set[int]:
    out: set[int] = set()
    for m in VREG.finditer(text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _valu_to_mfma_gaps(code: list[tuple[int, str, str]]) -> list[tuple[int, int]]:
    """(index, wait states) of every VALU instruction whose VGPR result a following MFMA of the same straight-line run
    reads as SrcA or SrcB, with fewer than MFMA_AB_WAIT wait states between them (each instruction between counts one,
    s_nop N counts N + 1).  The compiler keeps that distance for the code it can see; inline assembly is opaque to its
    hazard recognizer, so a VALU op written in asm can land closer and the MFMA then reads a stale operand."""
    bad = []
    for i, (_, mnem, ops) in enumerate(code):
        if not mnem.startswith("v_") or mnem.startswith(("v_mfma", "v_cmp", "v_readfirstlane", "v_readlane")):
            continue
        dst = _vgprs(ops.split("//")[0].split(",")[0])
        if not dst:
            continue
        waits = 0
        for _, m2, o2 in code[i + 1:i + 1 + MFMA_AB_WAIT + 1]:
            if m2.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
                break
            if m2.startswith("v_mfma"):
                srcs = o2.split("//")[0].split(",")
                if len(srcs) >= 3 and dst & (_vgprs(srcs[1]) | _vgprs(srcs[2])) and waits < MFMA_AB_WAIT:
                    bad.append((i, waits))
                break
            waits += int(o2.split()[0]) + 1 if m2 == "s_nop" and o2.split() else 1
            if waits >= MFMA_AB_WAIT:
                break
    return bad


def test_no_valu_result_reaches_an_mfma_operand_too_early(kernels):
    """Every kernel of the library (the ring and register-ring kernels once built their nibble unpack from an asm
    v_and_or_b32 that the scheduler placed one instruction ahead of the MFMA reading it: wrong products)."""
    checked = 0
    for name, code in kernels.items():
        assert not _valu_to_mfma_gaps(code), (name, _valu_to_mfma_gaps(code)[:4])
        checked += any(m.startswith("v_mfma") for _, m, _ in code)
    assert checked >= 50, f"expected the MFMA kernels, checked {checked}"


def test_valu_mfma_gap_check_rejects_a_planted_hazard():
    """Accepted with two instructions (or s_nop 1) between the write and the MFMA; rejected with one or none."""
    def prog(between: list[tuple[str, str]]) -> list[tuple[int, str, str]]:
        code = [("v_and_or_b32", "v44, v12, s68, v37")] + between + \
            [("v_mfma_f32_16x16x32_bf16", "v[52:55], v[56:59], v[44:47], v[52:55]"), ("s_endpgm", "")]
        return [(0x1000 + 4 * i, m, o) for i, (m, o) in enumerate(code)]

    nop = ("v_perm_b32", "v12, v11, v40, s67")
    assert not _valu_to_mfma_gaps(prog([nop, nop]))
    assert not _valu_to_mfma_gaps(prog([("s_nop", "1")]))
    assert _valu_to_mfma_gaps(prog([nop])) == [(0, 1)]
    assert _valu_to_mfma_gaps(prog([])) == [(0, 0)]
