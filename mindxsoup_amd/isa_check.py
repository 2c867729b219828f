"""Build-time check of the inline-asm global loads in compiled AMDGPU assembly.

The warp-specialized GEMM issues its NF4 loads as inline asm (csrc/common.h: gload_*), so the
compiler neither counts nor awaits them: the kernel waits by hand (s_waitcnt vmcnt) before it
uses a result and passes the value through vm_ready().  What the source cannot control is the
register allocator.  A copy or spill of a register whose load is still in flight reads stale
data, and a register given to another value while its load is in flight is overwritten when
the load lands.  This pass rules both out on the generated code.

Over each kernel's control-flow graph it tracks, for every VGPR written by an inline-asm load
(between the ``;;#ASMSTART`` / ``;;#ASMEND`` markers the compiler prints), how many vector
memory instructions the wave has issued since.  vmcnt counts in issue order, so
``s_waitcnt vmcnt(N)`` retires every load with N or more younger ones.  Where paths merge the
state keeps the youngest age of each register (a may-analysis, iterated to a fixed point), and
any instruction that names a register still pending on some path is reported.

    python -m mindxsoup_amd.isa_check file.s [symbol-prefix]
"""

import re
import sys

# vector memory instructions: each one counts in vmcnt (gfx9: stores too)
_VMEM = ("global_", "buffer_", "flat_", "scratch_")
_VGPR = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
_CAP = 64  # ages are capped: an old load stays pending until a wait retires it


def _vgprs(text):
    out = set()
    for m in _VGPR.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def functions(asm):
    """{symbol: [lines]} for every function in an assembly listing."""
    out = {}
    for name in re.findall(r"^\s*\.type\s+([^,\s]+),@function", asm, re.M):
        m = re.search(r"^" + re.escape(name) + r":", asm, re.M)
        if not m:
            continue
        end = asm.find(".Lfunc_end", m.end())
        out[name] = asm[m.end():end if end >= 0 else len(asm)].splitlines()
    return out


def _parse(lines):
    """Instructions as (text, inside_inline_asm) and label -> instruction index."""
    ins, labels, in_asm = [], {}, False
    for line in lines:
        if "#ASMSTART" in line:
            in_asm = True
        if "#ASMEND" in line:
            in_asm = False
        t = line.split(";")[0].strip()
        if not t:
            continue
        m = re.match(r"^([.\w$]+):", t)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        if t.startswith("."):
            continue  # directive
        ins.append((t, in_asm))
    return ins, labels


def _blocks(ins, labels):
    leaders = {0} | set(labels.values())
    for k, (t, _) in enumerate(ins):
        op = t.split()[0]
        if op.startswith(("s_branch", "s_cbranch")) or op in ("s_endpgm", "s_setpc_b64"):
            leaders.add(k + 1)
    leaders = sorted(x for x in leaders if x < len(ins))
    index = {b: n for n, b in enumerate(leaders)}
    spans = [(b, leaders[n + 1] if n + 1 < len(leaders) else len(ins))
             for n, b in enumerate(leaders)]
    succ = []
    for b, e in spans:
        t = ins[e - 1][0]
        op, args = t.split()[0], t.split()[1:]
        nxt = [index[e]] if e in index else []
        if op == "s_branch":
            succ.append([index[labels[args[0]]]])
        elif op.startswith("s_cbranch"):
            succ.append([index[labels[args[0]]]] + nxt)
        elif op in ("s_endpgm", "s_setpc_b64"):
            succ.append([])
        else:
            succ.append(nxt)
    _thread_known_conditions(ins, spans, succ)
    return spans, succ


_ZERO_MASK = re.compile(r"^s_mov_b64\s+(s\[\d+:\d+\]),\s*0$")
_TEST_MASK = re.compile(r"^s_and_b64\s+vcc,\s*exec,\s*(s\[\d+:\d+\])$")


def _thread_known_conditions(ins, spans, succ):
    """Drop the edges a zeroed lane mask rules out.

    The compiler joins paths through a flag block: each predecessor sets a mask
    (``s_mov_b64 s[a:b], 0`` or ``-1``) and jumps to ``s_and_b64 vcc, exec, s[a:b]`` +
    ``s_cbranch_vccz``/``vccnz``.  Coming from a predecessor that wrote 0, vcc is 0 and only one
    successor of the flag block is reachable; without this, that path would reach the other
    successor too and carry its loads there.  The predecessor's edge goes straight to the one
    successor (the flag block writes only scalar registers)."""
    for n, (b, e) in enumerate(spans):
        if len(succ[n]) != 1 or e - b < 1:
            continue
        last = ins[e - 1][0]
        k = e - 2 if last.startswith("s_branch") else e - 1
        m = _ZERO_MASK.match(ins[k][0]) if k >= b else None
        if not m:
            continue
        fb, fe = spans[succ[n][0]]
        if fe - fb != 2:
            continue
        t = _TEST_MASK.match(ins[fb][0])
        br = ins[fb + 1][0].split()
        if not t or t.group(1) != m.group(1) or br[0] not in ("s_cbranch_vccz", "s_cbranch_vccnz"):
            continue
        flag = succ[n][0]
        taken, fall = succ[flag][0], (succ[flag][1:] or [None])[0]
        nxt = taken if br[0] == "s_cbranch_vccz" else fall
        if nxt is not None:
            succ[n] = [nxt]


def _step(state, ins, b, e, report=None):
    st = dict(state)
    for k in range(b, e):
        text, in_asm = ins[k]
        op = text.split()[0]
        if op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", text)
            if m:
                n = int(m.group(1))
                st = {r: age for r, age in st.items() if age < n}
            continue
        operands = text[len(op):]
        if report is not None:
            hit = sorted(r for r in _vgprs(operands) if r in st)
            if hit:
                report.append((k, text, hit))
        if op.startswith(_VMEM):
            st = {r: min(age + 1, _CAP) for r, age in st.items()}
            if in_asm and "load" in op and "_lds" not in op:
                for r in _vgprs(operands.split(",")[0]):
                    st[r] = 0
    return st


def analyze(lines):
    """[(instruction index, text, pending VGPRs)] for one function's lines."""
    ins, labels = _parse(lines)
    if not ins:
        return []
    spans, succ = _blocks(ins, labels)
    state_in = [None] * len(spans)
    state_in[0] = {}
    work = [0]
    while work:
        n = work.pop()
        out = _step(state_in[n], ins, *spans[n])
        for m in succ[n]:
            old = state_in[m]
            new = dict(out) if old is None else dict(old)
            if old is not None:
                for r, age in out.items():
                    new[r] = min(age, new.get(r, _CAP + 1))
            if new != old:
                state_in[m] = new
                work.append(m)
    report = []
    for n, span in enumerate(spans):
        if state_in[n] is not None:
            _step(state_in[n], ins, *span, report)
    return report


def check(asm, prefix=""):
    """{symbol: report} for the functions whose symbol starts with `prefix` and that have
    findings; empty when the listing is clean."""
    bad = {}
    for name, lines in functions(asm).items():
        if name.startswith(prefix):
            rep = analyze(lines)
            if rep:
                bad[name] = rep
    return bad


def main(argv):
    asm = open(argv[1]).read()
    bad = check(asm, argv[2] if len(argv) > 2 else "")
    for name, rep in bad.items():
        print(f"{name}: {len(rep)} uses of registers with a load in flight")
        for k, text, regs in rep[:8]:
            print(f"   #{k}: {text}   pending {regs}")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
