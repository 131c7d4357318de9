"""Static check of the GEMM kernels' untracked global loads in compiled gfx950 assembly.

The GEMM issues its weight loads with inline asm so the compiler's conservative `s_waitcnt vmcnt(0)` at
loop back-edges cannot cancel the two-step prefetch; the kernel waits for them itself with explicit
`s_waitcnt vmcnt(N)` and ties the destination registers after the wait. The compiler does not know the
loads are still in flight, so a spill or a register reuse of such a destination before the wait lets
the late load overwrite an unrelated value (an address, in the faults this check was written for).

check_text() follows every control-flow path of each kernel (basic blocks, branches, loops, to a
fixpoint) and reports any instruction that reads or writes a destination VGPR of an inline-asm load
(between the ;;#ASMSTART / ;;#ASMEND markers) before an `s_waitcnt vmcnt(N)` that retires it, i.e.
with N smaller than the number of vector-memory instructions issued after that load."""
import re
import subprocess
from collections import defaultdict

VMEM_PREFIX = ("global_", "buffer_", "scratch_", "flat_")


def _regs(tok):
    tok = tok.strip().rstrip(",")
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return frozenset(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return frozenset([int(m.group(1))]) if m else frozenset()


def _blocks(body):
    blocks, cur, in_asm = [], ("entry", []), False
    for raw in body.split("\n")[1:]:
        if ";;#ASMSTART" in raw:
            in_asm = True
            continue
        if ";;#ASMEND" in raw:
            in_asm = False
            continue
        line = raw.split(";")[0].strip()
        m = re.match(r"(\.LBB\w+):", line)
        if m:
            blocks.append(cur)
            cur = (m.group(1), [])
            continue
        if not line or line.startswith("."):
            continue
        cur[1].append((line, in_asm))
        if line.split()[0].startswith(("s_cbranch", "s_branch")):
            # a branch ends its basic block; the code after it (unlabelled fall-through) is a new block
            blocks.append(cur)
            cur = (f"{cur[0]}+{len(blocks)}", [])
    blocks.append(cur)
    return blocks


def check_function(body):
    """Violations [(block label, index, instruction)] of one kernel's assembly text."""
    blocks = _blocks(body)
    idx = {b[0]: i for i, b in enumerate(blocks)}
    succ = defaultdict(list)
    for i, (_, ins) in enumerate(blocks):
        fall = True
        for line, _ in ins:
            op = line.split()[0]
            if op == "s_branch":
                succ[i].append(idx[line.split()[1]])
                fall = False
            elif op.startswith("s_cbranch"):
                succ[i].append(idx[line.split()[1]])
            elif op == "s_endpgm":
                fall = False
        if fall and i + 1 < len(blocks):
            succ[i].append(i + 1)
    state_in = {0: frozenset()}
    work, bad = [0], set()
    while work:
        i = work.pop()
        pend = set(state_in[i])  # (dest regs, load id, vector-memory ops issued since)
        for k, (line, in_asm) in enumerate(blocks[i][1]):
            op = line.split()[0]
            w = re.match(r"s_waitcnt\s+(?:.*?)vmcnt\((\d+)\)", line)
            if w:
                n = int(w.group(1))
                pend = {x for x in pend if x[2] < n}
                continue
            used = set()
            for a, b in re.findall(r"v\[(\d+):(\d+)\]", line):
                used |= set(range(int(a), int(b) + 1))
            used |= {int(x) for x in re.findall(r"\bv(\d+)\b", line)}
            for x in pend:
                if set(x[0]) & used:
                    bad.add((blocks[i][0], k, line))
            if op.startswith(VMEM_PREFIX):
                pend = {(x[0], x[1], min(x[2] + 1, 64)) for x in pend}
                if in_asm and "load" in op and "lds" not in op:
                    dst = _regs(line.split()[1])
                    if dst:
                        pend.add((dst, (i, k), 0))
        out = frozenset(pend)
        for s in succ[i]:
            old = state_in.get(s)
            new = out if old is None else old | out
            if new != old:
                state_in[s] = new
                work.append(s)
    return sorted(bad)


def check_text(text, name_filter="gemm_kernel"):
    """{kernel symbol: violations} for every kernel in an assembly file whose name contains name_filter."""
    out = {}
    for f in re.split(r"\n(?=_ZN\S*:)", text):
        name = f.split(":", 1)[0]
        if name_filter not in name:
            continue
        body = f[:f.find(".Lfunc_end")] if ".Lfunc_end" in f else f
        out[name] = check_function(body)
    return out


def compile_to_asm(src, out, include_dir, hipcc="/opt/rocm/bin/hipcc"):
    cmd = [hipcc, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-I", include_dir, "-o", out, src]
    subprocess.run(cmd, check=True, capture_output=True)
    return open(out).read()


def loop_depth_blocks(body):
    """[(label, loop depth, loop header, [instructions])] of one kernel's assembly, read from the compiler's
    loop comments on each block label (`in Loop: Header=BBx Depth=d`, `Inner Loop Header: Depth=d`; a
    loop header is its own loop's header; depth 0 and no header outside loops)."""
    out, lines = [], body.split("\n")
    for idx, raw in enumerate(lines):
        m = re.match(r"(\.LBB\w+|; %bb\.\d+):(.*)", raw)
        if m:
            notes = [m.group(2)]
            k = idx + 1
            while k < len(lines) and lines[k].strip().startswith(";"):  # continuation comment lines
                notes.append(lines[k])
                k += 1
            note = " ".join(notes)
            depths = [int(d) for d in re.findall(r"Depth=(\d+)", note)]
            if "Loop Header" in note:
                header = m.group(1).lstrip(".L")
            else:
                h = re.search(r"in Loop: Header=(BB\w+)", note)
                header = h.group(1) if h else None
            out.append((m.group(1), max(depths, default=0), header, []))
            continue
        line = raw.split(";")[0].strip()
        if out and line and not line.startswith(".") and not line.endswith(":"):
            out[-1][3].append(line)
    return out


def scratch_in_inner_mfma_loop(body):
    """Scratch (spill) accesses in the innermost loops that hold MFMAs: the K loop of a GEMM tile."""
    blocks = loop_depth_blocks(body)
    mfma = [(d, h) for _, d, h, ins in blocks if any(i.startswith("v_mfma") for i in ins)]
    if not mfma or max(d for d, _ in mfma) == 0:
        return []
    top = max(d for d, _ in mfma)
    loops = {h for d, h in mfma if d == top}
    return [(lab, i) for lab, d, h, ins in blocks if d == top and h in loops for i in ins if i.startswith("scratch_")]


def kernel_spills(text, name_filter):
    """{kernel symbol: (vgpr spill count, private segment bytes)} from the code-object metadata."""
    res = {}
    for block in re.split(r"\n\s+- \.", text):
        n = re.search(r"\.name:\s+(\S+)", block)
        s = re.search(r"\.vgpr_spill_count:\s+(\d+)", block)
        p = re.search(r"\.private_segment_fixed_size:\s+(\d+)", block)
        if n and s and p and name_filter in n.group(1):
            res[n.group(1)] = (int(s.group(1)), int(p.group(1)))
    return res
