"""Static checks on the gfx950 code objects this repository builds
(triton-metal_amd/lib/*.hsaco), read with the ROCm LLVM tools: the
clang-offload-bundler unbundles the device image, llvm-objdump prints its AMD
assembly, llvm-readelf its kernel metadata.

Used by tests/test_kernel_isa.py.  Nothing here runs on a GPU."""

import re
import subprocess
import tempfile
from functools import lru_cache
from pathlib import Path

import yaml

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "triton-metal_amd" / "lib"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def tools_present() -> bool:
    return all((LLVM / t).exists() for t in ("clang-offload-bundler", "llvm-objdump", "llvm-readelf"))


def images():
    return sorted(LIB.glob("*.hsaco"))


@lru_cache(maxsize=None)
def device_elf(image: Path) -> Path:
    out = Path(tempfile.mkdtemp(prefix="tm_isa_")) / (image.stem + ".elf")
    subprocess.run([str(LLVM / "clang-offload-bundler"), "--unbundle", "--type=o",
                    f"--targets={TARGET}", f"--input={image}", f"--output={out}"], check=True)
    return out


@lru_cache(maxsize=None)
def metadata(image: Path) -> dict:
    """name -> the kernel's amdhsa metadata map (vgpr_count, agpr_count,
    *_spill_count, private_segment_fixed_size, group_segment_fixed_size, ...)."""
    text = subprocess.run([str(LLVM / "llvm-readelf"), "--notes", str(device_elf(image))],
                          check=True, capture_output=True, text=True).stdout
    start = text.index("---")
    end = text.index("\n...", start)
    doc = yaml.safe_load(text[start:end])
    return {k[".name"]: k for k in doc["amdhsa.kernels"]}


_INSN = re.compile(r"^\s+(\S+)(.*?)//\s*([0-9A-Fa-f]+):")
_TARGET = re.compile(r"<([\w.]+)\+0x([0-9a-f]+)>")
_FUNC = re.compile(r"^([0-9a-f]+) <([\w.]+)>:")


@lru_cache(maxsize=None)
def disassembly(image: Path) -> dict:
    """name -> list of (address, mnemonic, operands, branch target address or None)."""
    text = subprocess.run([str(LLVM / "llvm-objdump"), "-d", "--no-show-raw-insn",
                           str(device_elf(image))], check=True, capture_output=True, text=True).stdout
    funcs, cur, starts = {}, None, {}
    for line in text.splitlines():
        m = _FUNC.match(line)
        if m:
            cur = m.group(2)
            starts[cur] = int(m.group(1), 16)
            funcs[cur] = []
            continue
        m = _INSN.match(line)
        if m and cur:
            target = None
            t = _TARGET.search(line)
            if t and m.group(1).startswith(("s_branch", "s_cbranch")):
                target = starts[t.group(1)] + int(t.group(2), 16)
            funcs[cur].append((int(m.group(3), 16), m.group(1), m.group(2).strip(), target))
    return funcs


def is_lds_dma(mnemonic: str, operands: str) -> bool:
    """A copy from global memory straight into LDS (buffer_load ... lds,
    global_load_lds_*)."""
    if mnemonic.startswith("global_load_lds_"):
        return True
    return mnemonic.startswith("buffer_load_") and re.search(r"\blds\b", operands) is not None


def is_vmem(mnemonic: str) -> bool:
    return mnemonic.startswith(("buffer_", "global_", "flat_", "scratch_"))


def vmcnt_wait(mnemonic: str, operands: str):
    """N of an `s_waitcnt vmcnt(N)`, or None."""
    if mnemonic != "s_waitcnt":
        return None
    m = re.search(r"vmcnt\((\d+)\)", operands)
    return int(m.group(1)) if m else None


def barriers_with_copy_in_flight(insns, depth=0):
    """Dataflow over the kernel's control-flow graph: the s_barrier
    instructions that some path reaches with an LDS copy that no vmcnt wait
    has covered and that has already crossed `depth` barriers.  vmcnt counts
    vector memory instructions in issue order, so `s_waitcnt vmcnt(N)` covers
    every copy followed by at least N later vector memory instructions.
    depth 0: every copy lands before the next barrier (a tile is published by
    the barrier after its copy); depth 1: before the second (three buffers in
    rotation, the copy of block j+2 in flight while block j is computed).  A
    violation would let a workgroup read a tile before this wave's part of it
    has landed."""
    if not insns:
        return []
    addrs = [a for a, *_ in insns]
    index = {a: i for i, a in enumerate(addrs)}
    leaders = {0}
    for i, (a, mn, ops, tgt) in enumerate(insns):
        if tgt is not None:
            leaders.add(index[tgt])
            if i + 1 < len(insns):
                leaders.add(i + 1)
        elif mn == "s_endpgm" and i + 1 < len(insns):
            leaders.add(i + 1)
    starts = sorted(leaders)
    blocks = [(s, (starts[k + 1] if k + 1 < len(starts) else len(insns))) for k, s in enumerate(starts)]
    block_of = {s: k for k, (s, _) in enumerate(blocks)}
    succ = []
    for s, e in blocks:
        a, mn, ops, tgt = insns[e - 1]
        out = []
        if tgt is not None:
            out.append(block_of[index[tgt]])
        if mn != "s_endpgm" and not mn.startswith("s_branch") and e < len(insns):
            out.append(block_of[e])
        succ.append(out)

    # state: a tuple over the copies that crossed 0, 1, ... depth barriers;
    # each entry None (no uncovered copy) or the fewest vector memory
    # instructions issued after the newest uncovered copy of that group
    def bump(k):
        return None if k is None else k + 1

    def step(state, mn, ops):
        if is_lds_dma(mn, ops):
            return (0,) + tuple(bump(k) for k in state[1:])
        if is_vmem(mn):
            return tuple(bump(k) for k in state)
        n = vmcnt_wait(mn, ops)
        if n is not None:
            return tuple(None if (k is not None and k >= n) else k for k in state)
        if mn == "s_barrier":
            return (None,) + state[:-1]
        return state

    def meet(x, y):
        return tuple(a if b is None else b if a is None else min(a, b) for a, b in zip(x, y))

    empty = (None,) * (depth + 1)
    state_in = [empty] * len(blocks)
    changed = True
    while changed:
        changed = False
        for k, (s, e) in enumerate(blocks):
            st = state_in[k]
            for a, mn, ops, tgt in insns[s:e]:
                st = step(st, mn, ops)
            for nk in succ[k]:
                new = meet(state_in[nk], st)
                if new != state_in[nk]:
                    state_in[nk] = new
                    changed = True
    bad = []
    for k, (s, e) in enumerate(blocks):
        st = state_in[k]
        for a, mn, ops, tgt in insns[s:e]:
            if mn == "s_barrier" and st[-1] is not None:
                bad.append(a)
            st = step(st, mn, ops)
    return bad
