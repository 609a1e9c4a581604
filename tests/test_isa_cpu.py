"""CPU checks of the instructions our own gfx950 build emits (the code object
compiled from this repository's kernels, read back with the ROCm LLVM tools).

1. Memory-model lowering. The split-K exchange of the W8A16 column-group
   kernels and the counted steps of the one-launch entries (kernels/phases.h)
   rely on three facts of the backend: a relaxed agent-scope atomic store is
   a global store with the sc1 cache policy (written through the XCD's L2),
   a relaxed agent-scope atomic load a global load with sc1, and neither
   brings L2-wide maintenance (buffer_wbl2 / buffer_inv). A probe kernel
   compiled with the production flags pins the first two; the production
   code object must hold no L2 maintenance at all and must use those
   stores and loads where the exchange lives. A compiler that lowered them
   otherwise fails here instead of computing wrong sums.
2. MFMA results read across a branch. A VALU read of an MFMA result needs
   wait states after the MFMA; the compiler places them inside a basic
   block, but one build sank a read past a conditional refill, so on the
   path that skipped it the read came one instruction after the last MFMA
   (element 3 of each fragment then varied from launch to launch). For
   every branch whose block ends in MFMAs, the wait states from each MFMA
   to the first read of its result at the branch target must be at least
   the fewest the compiler itself placed before such a read inside a block
   for that MFMA.
"""
import os
import re
import subprocess

import pytest

from lunaflux_amd import build as native_build

LLVM = "/opt/rocm/llvm/bin"
HIPCC = native_build.HIPCC
CODE_OBJECT = native_build.CODE_OBJECT

pytestmark = pytest.mark.skipif(
    not (os.path.exists(os.path.join(LLVM, "llvm-objdump")) and os.path.exists(HIPCC)
         and os.path.exists(CODE_OBJECT)),
    reason="needs the ROCm LLVM tools, hipcc and the built code object")


def disassemble(code_object, tmp):
    """{kernel: [(address, mnemonic, operands, (kernel, offset) of a branch
    target or None)]} from the disassembly of the gfx950 image of a code
    object built here."""
    elf = os.path.join(str(tmp), "fp8.elf")
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    f"--targets=hipv4-amdgcn-amd-amdhsa--{native_build.ARCH}", f"--input={code_object}",
                    f"--output={elf}"], check=True)
    text = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", f"--mcpu={native_build.ARCH}", elf],
                          check=True, capture_output=True, text=True).stdout
    out, cur = {}, None
    for line in text.split("\n"):
        m = re.match(r"^[0-9a-f]+ <(\w+)>:", line)
        if m:
            cur = out.setdefault(m.group(1), [])
            continue
        m = re.match(r"^\s+(\S+)\s*(.*?)\s*// ([0-9A-F]+):(?:[0-9A-F ]+)(?:<(\w+)\+0x([0-9a-f]+)>)?", line)
        if cur is None or not m:
            continue
        mnemonic, operands, addr = m.group(1), m.group(2), int(m.group(3), 16)
        target = None
        if mnemonic.startswith("s_cbranch") or mnemonic == "s_branch":
            tm = re.search(r"<(\w+)\+0x([0-9a-f]+)>", line)
            if tm:
                target = (tm.group(1), int(tm.group(2), 16))
        cur.append((addr, mnemonic, operands, target))
    assert len(out) > 50, "no kernels disassembled"
    return out


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    return disassemble(CODE_OBJECT, tmp_path_factory.mktemp("isa"))


def test_agent_scope_atomics_lower_to_write_through_accesses(tmp_path):
    src = tmp_path / "probe.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "extern \"C\" __global__ void probe(float *p, int *c, float v) {\n"
        "  __hip_atomic_store(p + threadIdx.x, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
        "  asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\");\n"
        "  const int before = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
        "  p[64 + threadIdx.x] = __hip_atomic_load(p + 128 + threadIdx.x + before, __ATOMIC_RELAXED,\n"
        "                                          __HIP_MEMORY_SCOPE_AGENT);\n"
        "}\n")
    asm = tmp_path / "probe.s"
    subprocess.run([HIPCC, "--genco", *native_build.DEVICE_FLAGS, "-S", str(src), "-o", str(asm)],
                   check=True, capture_output=True)
    body = [l.strip() for l in asm.read_text().split("\n") if re.match(r"\s+(global_|buffer_)", l)]
    stores = [l for l in body if l.startswith("global_store_dword")]
    loads = [l for l in body if l.startswith("global_load_dword")]
    assert any(l.endswith(" sc1") for l in stores), body     # the atomic store
    assert any(not re.search(r"\bsc[01]\b", l) for l in stores), body  # the plain store
    assert loads and all(l.endswith(" sc1") for l in loads), body
    assert any(l.startswith("global_atomic_add") for l in body), body
    assert not any(l.startswith(("buffer_wbl2", "buffer_inv")) for l in body), body


def test_no_l2_maintenance_and_write_through_exchange(kernels):
    for name, ins in kernels.items():
        assert not any(m.startswith(("buffer_wbl2", "buffer_inv", "buffer_wbinvl1")) for _, m, _, _ in ins), name
    # the split-K column-group kernels: partials stored and loaded through
    # sc1, the arrival counted with an atomic add
    for name in ("lf_fp8_w8a16_dense_m32", "lf_fp8_w8a16_gate_up_b128_m64", "lf_fp8_w8a16_dense_k14336_m32"):
        ins = kernels[name]
        assert any(m.startswith("global_store_dword") and ops.endswith("sc1") for _, m, ops, _ in ins), name
        assert any(m.startswith("global_load_dword") and ops.endswith("sc1") for _, m, ops, _ in ins), name
        assert any(m == "global_atomic_add" for _, m, _, _ in ins), name


def _regs(token):
    """Register numbers ('a', n) / ('v', n) of an operand token."""
    m = re.match(r"([av])\[(\d+):(\d+)\]$", token)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([av])(\d+)$", token)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _operands(ops):
    return [t.strip() for t in re.split(r",\s*", ops) if t.strip()]


def _waits(mnemonic, ops):
    if mnemonic == "s_nop":
        return int(ops, 0) + 1
    return 1


def _reads(mnemonic, ops):
    """Registers a VALU instruction reads (sources), MFMAs excluded (their
    accumulator chains are interlocked)."""
    if not mnemonic.startswith("v_") or mnemonic.startswith("v_mfma"):
        return set()
    toks = _operands(ops)
    out = set()
    for t in toks[1:]:
        out |= _regs(t)
    return out


def test_mfma_results_are_not_read_early_across_branches(kernels):
    flagged = early_mfma_reads(kernels)
    assert not flagged, "\n".join(flagged[:20])


def early_mfma_reads(kernels):
    # fewest wait states the compiler places, inside a block, between each
    # MFMA opcode and the first VALU read of its result
    inblock = {}
    for name, ins in kernels.items():
        for i, (_, m, ops, _) in enumerate(ins):
            if not m.startswith("v_mfma"):
                continue
            dst = _regs(_operands(ops)[0])
            w = 0
            for _, m2, ops2, tgt in ins[i + 1:i + 40]:
                if tgt is not None or m2.startswith("s_cbranch") or m2 == "s_branch" or m2 == "s_endpgm":
                    break
                if dst & _reads(m2, ops2):
                    inblock[m] = min(inblock.get(m, 99), w)
                    break
                if m2.startswith("v_mfma") and dst & _regs(_operands(ops2)[0]):
                    break  # overwritten by another MFMA first
                w += _waits(m2, ops2)
    assert inblock, "no in-block MFMA result reads found"
    flagged = []
    for name, ins in kernels.items():
        index = {a: i for i, (a, *_) in enumerate(ins)}
        base = ins[0][0]
        for i, (addr, m, ops, tgt) in enumerate(ins):
            if tgt is None or tgt[0] != name:
                continue
            # MFMAs among the last instructions of the branch's block
            pending = []
            w = 1  # the branch itself
            for _, m2, ops2, t2 in reversed(ins[max(0, i - 16):i]):
                if t2 is not None or m2 == "s_endpgm":
                    break
                if m2.startswith("v_mfma"):
                    pending.append((m2, _regs(_operands(ops2)[0]), w))
                w += _waits(m2, ops2)
            if not pending:
                continue
            j = index.get(base + tgt[1])
            if j is None:
                continue
            fwd = 0
            for _, m3, ops3, t3 in ins[j:j + 40]:
                reads = _reads(m3, ops3)
                hit = [(mm, d) for mm, regs, d in pending if regs & reads]
                if hit:
                    for mm, d in hit:
                        need = inblock.get(mm, 8)
                        if d + fwd < need:
                            flagged.append(f"{name}+{addr - base:#x}: {m3} {ops3} {d + fwd} < {need} after {mm}")
                    break
                if t3 is not None or m3 == "s_endpgm":
                    break
                fwd += _waits(m3, ops3)
    return flagged
