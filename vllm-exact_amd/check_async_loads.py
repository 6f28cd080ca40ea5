"""Build-time check of the inline asm in exact_gemm_xw.hip (direct-to-LDS copies that set M0)
and of any load issued from inline asm.

    python3 check_async_loads.py KERNEL.s [kernel-name-substring]

The compiler does not know that an inline-asm `global_load_dwordx4` writes its destination
registers only when the data arrives; it treats them as written at the asm statement. The
kernel keeps every such destination live until an explicit `s_waitcnt vmcnt(N)` covers the
load. This script proves that on the generated gfx950 assembly: it walks every control-flow
path from each inline-asm load, counting the memory instructions issued after it, and fails
if any instruction reads or writes one of the load's destination VGPRs before an
`s_waitcnt vmcnt(N)` with N <= that count (the load is then complete), or if a path reaches
`s_endpgm` first. It also fails if compiler-generated code in a checked kernel uses M0, which
the kernels' inline asm writes. Exit status 0: every inline-asm load is safe; 1: a violation
(printed).
"""
import re
import sys

MEMORY_OPS = ("global_", "buffer_", "flat_", "scratch_")


def vgprs(text):
    """VGPR numbers named in an operand string (v7, v[4:7]); AGPRs and SGPRs are ignored."""
    out = set()
    for m in re.finditer(r"(?<![a-z_])v\[(\d+):(\d+)\]|(?<![a-z_\[])v(\d+)\b", text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def parse(body):
    """Instructions of one function as (text, from_inline_asm) and its label positions."""
    insts, labels, in_asm = [], {}, False
    for raw in body.split("\n")[1:]:
        line = raw.strip()
        if line.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if line.startswith(";;#ASMEND"):
            in_asm = False
            continue
        line = line.split(";")[0].strip()
        if not line:
            continue
        if re.match(r"^\.LBB\S+:$", line):
            labels[line[:-1]] = len(insts)
            continue
        if line.startswith("."):
            continue
        insts.append((line, in_asm))
    return insts, labels


def check_function(name, body):
    insts, labels = parse(body)

    def successors(i):
        parts = insts[i][0].split()
        if parts[0] == "s_endpgm":
            return []
        if parts[0] == "s_branch":
            return [labels[parts[1]]]
        if parts[0].startswith("s_cbranch"):
            return [labels[parts[1]], i + 1]
        return [i + 1] if i + 1 < len(insts) else []

    loads = violations = 0
    # M0 is written by the kernel's inline asm (the LDS address of its direct-to-LDS copies):
    # the compiler's own code in the same function must not use it
    for text, from_asm in insts:
        if not from_asm and re.search(r"\bm0\b", text):
            violations += 1
            print(f"{name}: compiler-generated use of m0: {text}")
    for i, (text, from_asm) in enumerate(insts):
        if not (from_asm and text.startswith("global_load_dwordx4 ")):
            continue
        loads += 1
        dst = vgprs(text.split(None, 1)[1].split(",")[0])
        stack, seen, bad = [(j, 0) for j in successors(i)], set(), None
        while stack and bad is None:
            j, younger = stack.pop()
            while True:
                key = (j, min(younger, 64))
                if key in seen:
                    break
                seen.add(key)
                cur = insts[j][0]
                op = cur.split()[0]
                if op == "s_waitcnt":
                    m = re.search(r"vmcnt\((\d+)\)", cur)
                    if m and younger >= int(m.group(1)):
                        break  # the load has completed on this path
                elif op == "s_endpgm":
                    bad = f"reaches s_endpgm uncovered: {text}"
                    break
                else:
                    args = cur.split(None, 1)[1] if " " in cur else ""
                    if vgprs(args) & dst:
                        bad = f"{text}  ||  {cur}"
                        break
                    if op.startswith(MEMORY_OPS):
                        younger += 1
                nxt = successors(j)
                if not nxt:
                    break
                stack.extend((k, younger) for k in nxt[1:])
                j = nxt[0]
        if bad is not None:
            violations += 1
            print(f"{name}: {bad}")
    return loads, violations


def main():
    path = sys.argv[1]
    pattern = sys.argv[2] if len(sys.argv) > 2 else ""
    asm = open(path).read()
    names = [n for n in re.findall(r"^(_Z\S+):", asm, re.M) if pattern in n]
    total_loads = total_bad = 0
    for name in names:
        body = asm[asm.index(name + ":"):]
        body = body[:body.index(".Lfunc_end")]
        loads, bad = check_function(name, body)
        total_loads += loads
        total_bad += bad
    print(f"check_async_loads: {len(names)} kernels, {total_loads} inline-asm loads, {total_bad} violations")
    sys.exit(1 if total_bad or not names else 0)


if __name__ == "__main__":
    main()
