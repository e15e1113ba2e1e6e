"""Checks on the gfx950 code the library was built into (our own build, disassembled with ROCm's llvm-objdump): the
kernels that stream K slices into LDS with direct-to-LDS loads wait for them with `s_waitcnt vmcnt(N)`, N > 0, so
that later loads may stay in flight.  That is only correct while the instruction order the counts assume holds:

* w4_big_kernel (prefill, two register sets): the N loads after the last x load of a slice are the next weight
  fetch, so at least N vector-memory loads must follow the last `global_load_lds` before each such wait;
* mm_ring_kernel (W8A8 small M, S-stage ring): each loop iteration issues exactly the NI direct-to-LDS loads of one
  slice and no other vector-memory load, and waits with vmcnt((S - 2) * NI) ("slice kt + 1 has landed");
* w4_ring_kernel (W4 on the CDNA4 layout, 33..64 rows or long K): the same rule with NI = 4 MB / BW + T + 2 buffer
  loads into LDS per step.

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


def _check_ring_loops(name: str, code: list[tuple[int, str, str]], ni: int, s: int) -> int:
    """Every barrier wait of a ring kernel is vmcnt((S - 2) * NI), and the loop around it issues exactly NI
    direct-to-LDS loads and no other vector-memory load.  Returns the loops checked."""
    addr = {a: i for i, (a, _, _) in enumerate(code)}
    waits = _barrier_waits(code)
    assert waits and all(n == (s - 2) * ni for _, n in waits), (name, waits, ni, s)
    found = 0
    for wi, _ in waits:
        # the loop around this wait: the first later branch whose target lies before the wait
        for j in range(wi + 1, len(code)):
            mnem, ops = code[j][1], code[j][2]
            if mnem.startswith(("s_cbranch", "s_branch")):
                tgt = re.search(r"<\S+\+0x([0-9a-f]+)>", ops)
                base = code[0][0]
                if tgt and base + int(tgt.group(1), 16) <= code[wi][0]:
                    head = addr[base + int(tgt.group(1), 16)]
                    body = code[head:j + 1]
                    dma = sum(1 for _, m, o in body if _lds_dma(m, o))
                    other = sum(1 for _, m, o in body if _vmem(m) and not _lds_dma(m, o))
                    assert dma == ni and other == 0, f"{name}: loop issues {dma} DMA + {other} other loads"
                    found += 1
                    break
    return found


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
