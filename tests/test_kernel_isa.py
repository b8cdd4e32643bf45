"""Properties of the compiled gfx950 code that GPU runs cannot pin down
reliably (CPU only: hipcc cross-compiles, nothing is launched).

The attention kernel fills LDS with global_load_lds (DMA counted by vmcnt)
and reads it with inline-assembly ds_read instructions after a workgroup
barrier. Nothing at the barrier waits for loads by itself, so each barrier
must be preceded, in its own basic block or one that falls through into it,
by an explicit s_waitcnt vmcnt(n)
with no LDS DMA issued between that wait and the barrier; otherwise a wave
may read a tile before its DMA has landed, a timing-dependent error in the
attention output. n may leave the DMA of the next step in flight (the K and
V DMA of one tile: 4 instructions per wave of an 8-wave workgroup), which
was sent after the tile the step reads; loads complete in order.

The GEMM and attention kernels read their MFMA operand fragments with
inline-assembly ds_read pairs, whose data the compiler takes to be there at
once: no instruction may name a register such a read will still write.
"""

from __future__ import annotations

import functools
import os
import re
import subprocess
import tempfile

import pytest

from opengenie_amd import build

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "opengenie_amd", "csrc")


@functools.lru_cache(maxsize=None)
def _device_asm(src: str) -> str:
    """The device assembly of src; the same source must also assemble (-S
    alone does not check inline-assembly operands such as offset ranges)."""
    flags = [f for f in build.HIPCC_FLAGS if f not in ("-fPIC", "-Wall", "-Wno-unused-function")]
    with tempfile.TemporaryDirectory() as td:
        out = os.path.join(td, "k.s")
        for mode, path in (("-S", out), ("-c", os.path.join(td, "k.o"))):
            res = subprocess.run([build.hipcc(), *flags, "--cuda-device-only", mode, "-o", path, src],
                                 capture_output=True, text=True)
            assert res.returncode == 0, res.stderr[-2000:]
        return open(out).read()


def _kernel_body(asm: str, kernel_substr: str) -> list[str]:
    lines = asm.splitlines()
    start = next(i for i, l in enumerate(lines) if re.match(r"^_Z\w*" + kernel_substr + r"\w*:", l))
    end = next(i for i in range(start, len(lines)) if lines[i].strip().startswith(".Lfunc_end"))
    return [l.split(";")[0].strip() for l in lines[start + 1:end]]


def barrier_violations(body: list[str], max_vmcnt: int = 0) -> list[int]:
    """Indexes of s_barrier instructions not preceded, within their basic
    block or the blocks that fall through into it, by s_waitcnt
    vmcnt(n <= max_vmcnt) with no LDS DMA after it. A block without a label
    is entered only by falling through, so the scan goes on past the
    conditional branch that ends the block before it; a label (a jump
    target) or an unconditional branch ends it."""
    bad = []
    for i, ins in enumerate(body):
        if ins != "s_barrier":
            continue
        ok = False
        for j in range(i - 1, -1, -1):
            prev = body[j]
            if prev.endswith(":") or prev.startswith("s_branch"):
                break  # a block other code can jump into
            if "load_lds" in prev:
                break
            m = re.search(r"\bvmcnt\((\d+)\)", prev) if prev.startswith("s_waitcnt") else None
            if m:
                ok = int(m.group(1)) <= max_vmcnt
                break
        if not ok:
            bad.append(i)
    return bad


def test_barrier_check_sees_a_missing_wait():
    body = ["global_load_lds_dwordx4 v1, s[2:3]", "s_waitcnt lgkmcnt(0)", "s_barrier"]
    assert barrier_violations(body) == [2]
    body = [".LBB0_1:", "s_waitcnt vmcnt(0)", ".LBB0_2:", "s_barrier"]
    assert barrier_violations(body) == [3]
    body = ["s_waitcnt vmcnt(0)", "global_load_lds_dwordx4 v1, s[2:3]", "s_barrier"]
    assert barrier_violations(body) == [2]
    body = ["global_load_lds_dwordx4 v1, s[2:3]", "s_waitcnt vmcnt(0)", "v_mov_b32 v0, 0", "s_barrier"]
    assert barrier_violations(body) == []
    body = ["s_waitcnt vmcnt(4)", "s_barrier"]
    assert barrier_violations(body) == [1] and barrier_violations(body, 4) == []
    assert barrier_violations(["s_waitcnt vmcnt(8)", "s_barrier"], 4) == [1]


def test_barrier_check_follows_fall_through_only():
    """A wait before a conditional branch covers the barrier of the block the
    branch falls through to, not one behind a jump target."""
    through = ["global_load_lds_dwordx4 v1, s[2:3]", "s_waitcnt vmcnt(0)", "s_cbranch_scc0 .LBB0_9", "",
               "v_mov_b32_e32 v0, v1", "s_barrier"]
    assert barrier_violations(through) == []
    target = ["global_load_lds_dwordx4 v1, s[2:3]", "s_waitcnt vmcnt(0)", "s_cbranch_scc0 .LBB0_9",
              ".LBB0_8:", "s_barrier"]
    assert barrier_violations(target) == [4]
    after_dma = ["s_waitcnt vmcnt(0)", "s_cbranch_scc0 .LBB0_9", "global_load_lds_dwordx4 v1, s[2:3]", "s_barrier"]
    assert barrier_violations(after_dma) == [3]


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc") and not os.environ.get("HIPCC"),
                    reason="hipcc not present")
def test_attention_barriers_wait_for_lds_dma():
    """Both instances of the bf16 kernel: 8 waves with three tile pairs (the
    wait may leave the next step's 4 DMA instructions in flight) and 4 waves
    with two pairs (nothing may stay in flight: the next DMA goes into the
    pair the step after reads)."""
    asm = _device_asm(os.path.join(CSRC, "attention.hip"))
    seen = set()
    for mangled, max_vmcnt in (("k_attentionILi8ELi3EE", 4), ("k_attentionILi4ELi2EE", 0)):
        body = _kernel_body(asm, mangled)
        seen.add(mangled)
        n_barriers = sum(1 for ins in body if ins == "s_barrier")
        assert n_barriers >= 2, mangled
        assert any("load_lds" in ins for ins in body), mangled
        assert barrier_violations(body, max_vmcnt=max_vmcnt) == [], mangled
    assert len(seen) == 2


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc") and not os.environ.get("HIPCC"),
                    reason="hipcc not present")
def test_fp8_attention_barriers_wait_for_lds_dma():
    """The FP8 kernel sends two DMA instructions per wave and step (the K
    tile and the V^T tile), so the wait may leave the next step's two in flight."""
    body = _kernel_body(_device_asm(os.path.join(CSRC, "attention.hip")), "k_attention_fp8")
    assert sum(1 for ins in body if ins == "s_barrier") >= 2
    assert any("load_lds" in ins for ins in body)
    assert barrier_violations(body, max_vmcnt=2) == []


# ----------------------------------------------------------------- LDS reads
_LDS_RESULT = ("ds_read", "ds_load", "ds_bpermute", "ds_permute", "ds_swizzle")


def _vregs(text: str) -> set:
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if m.group(1) is not None:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def lds_read_hazards(body: list[str]) -> list[int]:
    """Indexes of instructions that name a VGPR an LDS read still in flight
    will write: the read's data returns after later instructions issue, so
    such a register may be read before the data lands, or overwritten by it
    afterwards. s_waitcnt lgkmcnt(n) retires all but the newest n LDS
    operations (LDS operations complete in order); the check runs through
    each straight-line stretch (an unconditional branch ends one). The
    compiler places its own waits for the LDS reads it sees; inline-assembly
    reads are the kernel's to wait for, and a multi-instruction asm block
    with outputs that are not early-clobber can hand the first read's
    destination to the second read as its address."""
    pending: list[set] = []
    bad = []
    for i, ins in enumerate(body):
        if not ins or ins.startswith("."):
            continue
        op, _, args = ins.partition(" ")
        if op.endswith(":"):
            continue
        if op in ("s_branch", "s_endpgm", "s_setpc_b64"):
            pending = []
            continue
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", args)
            if m:
                del pending[:max(0, len(pending) - int(m.group(1)))]
            continue
        busy = set().union(*pending) if pending else set()
        if op.startswith("ds_"):
            ops = [a.strip() for a in re.split(r",(?![^\[]*\])", args)]
            returns = op.startswith(_LDS_RESULT) or "_rtn" in op
            dst = _vregs(ops[0]) if returns else set()
            srcs = set().union(*(_vregs(o) for o in (ops[1:] if returns else ops)))
            if (srcs | dst) & busy:
                bad.append(i)
            pending.append(dst)
        elif op.startswith(("s_load", "s_buffer_load")):
            pending.append(set())  # also counted by lgkmcnt
        elif _vregs(args) & busy:
            bad.append(i)
    return bad


def test_lds_read_hazard_check_sees_both_mistakes():
    # the first read's destination is the second read's address
    body = ["ds_read_b128 v[2:5], v2 offset:0", "ds_read_b128 v[6:9], v3 offset:0", "s_waitcnt lgkmcnt(0)"]
    assert lds_read_hazards(body) == [1]
    body = ["ds_read_b128 v[10:13], v2 offset:0", "ds_read_b128 v[14:17], v3 offset:0", "s_waitcnt lgkmcnt(0)",
            "v_add_f32_e32 v0, v10, v14"]
    assert lds_read_hazards(body) == []
    # a use before the wait, and one that the wait of the newest read leaves open
    body = ["ds_read_b64 v[4:5], v1", "v_mov_b32_e32 v6, v4", "s_waitcnt lgkmcnt(0)"]
    assert lds_read_hazards(body) == [1]
    body = ["ds_read_b64 v[4:5], v1", "ds_read_b64 v[8:9], v1 offset:8", "s_waitcnt lgkmcnt(1)",
            "v_mov_b32_e32 v6, v4", "v_mov_b32_e32 v7, v8"]
    assert lds_read_hazards(body) == [4]
    body = ["ds_read_b64 v[4:5], v1", "s_branch .LBB0_2", ".LBB0_1:", "v_mov_b32_e32 v4, 0"]
    assert lds_read_hazards(body) == []


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc") and not os.environ.get("HIPCC"),
                    reason="hipcc not present")
@pytest.mark.parametrize("src", ["fp8_gemm.hip", "attention.hip"])
def test_no_register_of_an_outstanding_lds_read_is_named(src):
    """Every kernel of the two sources that read LDS through inline assembly
    (the other sources leave their LDS reads to the compiler, which waits for
    them itself): no instruction names a register that an LDS read still in
    flight will write. For the operand fragments this needs the
    early-clobber outputs of their two-read asm."""
    asm = _device_asm(os.path.join(CSRC, src))
    lines = asm.splitlines()
    kernels = [i for i, l in enumerate(lines) if re.match(r"^_Z\w+:", l) and ".amdhsa" not in l]
    assert kernels
    checked = 0
    for start in kernels:
        end = next((i for i in range(start, len(lines)) if lines[i].strip().startswith(".Lfunc_end")), None)
        if end is None:
            continue
        body = [l.split(";")[0].strip() for l in lines[start + 1:end]]
        assert lds_read_hazards(body) == [], (src, lines[start])
        checked += 1
    assert checked >= 1
