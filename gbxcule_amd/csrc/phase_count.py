"""Static instruction counts of the step kernel's hot loop, phase by phase.

Copies the kernel sources to a temporary directory, inserts assembler
comments at the phase boundaries of the loop (fetch, bus reads, datapath,
next-record load, write phase, fast tail, loop back edge) and at the head of
each block the loop hints as rare, compiles the device code for gfx950 to
assembly and walks ``step_kernel<ROM_ONLY, no debug, no cart RAM>`` along the compiler's
fall-through layout: an unconditional branch is followed, a conditional
branch falls through, except an ``s_cbranch_execz`` whose skipped region
opens with a rare-block marker, which is taken (no lane runs the rare block).
The markers are comments, so the instruction stream compiles as without them
(the kernel sizes with and without are printed).

    python gbxcule_amd/csrc/phase_count.py [--out FILE]
"""

from __future__ import annotations

import argparse
import re
import subprocess
import sys
import tempfile
from pathlib import Path

CSRC = Path(__file__).resolve().parent
INCLUDE = CSRC.parent.parent / "include"
sys.path.insert(0, str(CSRC.parent))
from build import DEVICE_FLAGS  # noqa: E402  (the flags the library is built with)
KERNEL = "_ZN3gbx12_GLOBAL__N_111step_kernelILi0ELb0ELb0E"  # step_kernel<MBC_ROM_ONLY, false, false>
PHASES = ("fetch", "bus", "exec", "nextrec", "write", "tail", "loop")
LABELS = {
    "fetch": "fetch (record valid check)",
    "bus": "bus reads (address, load, fix-ups)",
    "exec": "datapath (exec_insn)",
    "nextrec": "next pc, next record load",
    "write": "write phase",
    "tail": "fast tail (budget test, counters)",
    "loop": "loop condition, back edge",
}


def _insert(src: str, anchor: str, text: str, after: bool = False) -> str:
    i = src.index(anchor)
    j = i + len(anchor) if after else i
    return src[:j] + text + src[j:]


def _rare(src: str, anchor: str) -> str:
    """A rare-block marker right after the '{' that opens the block at anchor."""
    j = src.index("{", src.index(anchor))
    return src[: j + 1] + ' asm volatile(";@rare");' + src[j + 1 :]


def marked_sources(dst: Path) -> None:
    step = (CSRC / "gbx_step.hip").read_text()
    m = lambda name: f'asm volatile(";@phase {name}");\n'  # noqa: E731
    step = _insert(step, "      // ---- fetch + decode", m("fetch"))
    step = _insert(step, "      // ---- bus reads", m("bus"))
    step = _insert(step, "      // ---- execute (gbx_exec.h)", m("exec"))
    step = _insert(step, "      L.pc = npc;\n      // fetch the next record", m("nextrec"))
    step = _insert(step, "    // ---- write phase, debug checks", m("write"))
    step = _insert(step, "    const uint32_t lc_now = L.lcdc;", m("tail"))
    step = _insert(step, "      L.budget -= cycles;\n", m("loop"), after=True)
    step = _insert(step, "  instr += ninstr;\n  cyc += ncyc;\n\n  // ---- post-step", m("exit"))
    step = step.replace("if (__builtin_expect(__ballot(fx) != 0u, 0)) v = fx ? read_ppu(x, v) : v;",
                        "if (__builtin_expect(__ballot(fx) != 0u, 0)) { v = fx ? read_ppu(x, v) : v; }")
    for anchor in (
        "if (__builtin_expect(__ballot(fx) != 0u, 0))",  # STAT and deferred-LY read fix-up
        "if (__builtin_expect((!plain_store(x0)) | (two & !plain_ram(x1)), 0))",  # IO/MBC writes
        "if (__builtin_expect(__ballot(!rv) != 0u, 0))",  # fetch outside the record windows
        "if (__builtin_expect(nr > 1u, 0))",  # second read byte (POP, RET)
        "if (__builtin_expect(__ballot(o.misc != 0u) != 0u, 0))",  # DI/EI/HALT/traps, poll/copy loops
        "    } else {\n      L.settle();\n      cycles = L.halt_cycles(cframe);",  # halted lanes
        "    } else if (!trap) {\n      L.settle();\n      L.timer_tick(cycles);",  # full timer/PPU/IRQ sequence
    ):
        step = _rare(step, anchor)
    exe = (CSRC / "gbx_exec.h").read_text()
    daa = "if (__builtin_expect((FL & (1u << 30)) != 0u, 0)) {"
    exe = exe.replace(daa, daa + ' asm volatile(";@rare");')
    for f in CSRC.iterdir():
        if f.suffix in (".h", ".hip"):
            (dst / f.name).write_text(f.read_text())
    (dst / "gbx_step.hip").write_text(step)
    (dst / "gbx_exec.h").write_text(exe)


def assemble(src: Path, out: Path) -> list[str]:
    subprocess.run(
        ["/opt/rocm/bin/hipcc", *DEVICE_FLAGS, "--cuda-device-only", "-S", "-I", str(INCLUDE), "-o", str(out),
         str(src)],
        check=True, stderr=subprocess.DEVNULL)
    lines = out.read_text().split("\n")
    st = next(i for i, x in enumerate(lines) if x.startswith(KERNEL))
    en = next(i for i in range(st, len(lines)) if lines[i].startswith((".Lfunc_end", "; Kernel info")))
    return lines[st:en]


def kind(op: str) -> str:
    if op.startswith("v_"):
        return "VALU"
    if op.startswith(("s_cbranch", "s_branch")):
        return "branch"
    if op.startswith(("s_waitcnt", "s_nop")):
        return "wait/nop"
    if op.startswith("s_"):
        return "SALU"
    if op.startswith(("global_", "buffer_", "flat_", "scratch_")):
        return "VMEM"
    return "other"


def parse(body: list[str]):
    ins, labels = [], {}
    for raw in body:
        s = raw.strip()
        lm = re.match(r"^([.\w$]+):", s)
        if lm:
            labels[lm.group(1)] = len(ins)
            continue
        if not s or s[0] in ".#" or (s[0] == ";" and not s.startswith((";@phase", ";@rare"))):
            continue
        ins.append(s)
    return ins, labels


def walk(ins: list[str], labels: dict[str, int]) -> dict[str, dict[str, int]]:
    starts = set(labels.values())
    marks = {m.group(1): i for i, s in enumerate(ins) if (m := re.match(r";@phase (\w+)", s))}
    out = {}
    for name, i in marks.items():
        counts: dict[str, int] = {}
        j, seen = i + 1, set()
        while j < len(ins) and j not in seen:
            seen.add(j)
            s = ins[j]
            if s == ";@rare":
                j += 1
                continue
            if s.startswith(";@phase"):
                break
            op = s.split()[0]
            counts[kind(op)] = counts.get(kind(op), 0) + 1
            if op == "s_branch":
                j = labels[s.split()[1]]
                continue
            if op == "s_cbranch_execz":
                tgt = labels[s.split()[1]]
                k, head = j + 1, []
                while k < tgt and k not in starts and not ins[k].startswith(("s_cbranch", "s_branch")):
                    head.append(ins[k])
                    k += 1
                if tgt > j and ";@rare" in head:
                    j = tgt
                    continue
            if op == "s_endpgm":
                break
            j += 1
        out[name] = counts
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", type=Path, default=None)
    args = ap.parse_args()
    with tempfile.TemporaryDirectory() as td:
        d = Path(td)
        marked_sources(d)
        mk = assemble(d / "gbx_step.hip", d / "marked.s")
        pl = assemble(CSRC / "gbx_step.hip", d / "plain.s")
    size = lambda b: sum(1 for x in b if (s := x.strip()) and s[0] not in ";.#" and not re.match(r"^[.\w$]+:", s))  # noqa: E731
    res = walk(*parse(mk))
    cols = ("VALU", "SALU", "branch", "VMEM", "wait/nop")
    L = ["# Step kernel hot loop, static instructions per phase (gfx950, step_kernel<ROM_ONLY, no debug, no cart RAM>)",
         f"Command: python gbxcule_amd/csrc/phase_count.py  (kernel size {size(pl)} instructions as built, "
         f"{size(mk)} with the phase markers)", "",
         "| Phase | " + " | ".join(cols) + " | all |", "|---" * (len(cols) + 2) + "|"]
    tot = dict.fromkeys(cols, 0)
    for p in PHASES:
        c = res.get(p, {})
        for k in cols:
            tot[k] += c.get(k, 0)
        L.append(f"| {LABELS[p]} | " + " | ".join(str(c.get(k, 0)) for k in cols) + f" | {sum(c.values())} |")
    L.append("| **one loop iteration** | " + " | ".join(f"**{tot[k]}**" for k in cols) + f" | **{sum(tot.values())}** |")
    L += ["", "Rare blocks (skipped when no lane runs them): DIV/TIMA/STAT/LY read fix-up, IO/MBC writes, fetch outside the "
          "record windows, the second read byte, DI/EI/HALT/trap and poll/copy fast-forward, halted lanes, the full "
          "timer/PPU/interrupt sequence, DAA."]
    text = "\n".join(L) + "\n"
    if args.out:
        args.out.write_text(text)
    sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
