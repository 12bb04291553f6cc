"""Extract the structure of the reference's three other golden kernels into
a JSON fixture (run where /root/reference exists; the fixture is committed).

Sources, the reference's blessed emitter output for the kernels of its
tests/test_msl_snapshots.py:34-110:
- tests/golden/conditional_loop.metal: scan body ops, trip count, block size;
- tests/golden/blocked_saxpy.metal: per-operand offset (program id x stride),
  block size, elementwise ops;
- tests/golden/copy_2d.metal: offsets, element count, copy direction.

Facts recorded per kernel:
- "offsets": operand -> list of [grid axis, stride] terms (empty = base);
- "elements": elements per operand block;
- "ops": [primitive, operands...] in emission order, operands normalised to
  operand names ("in0", "in1", ...), the loop carry "carry", literals as
  float strings, "e<k>" for the k-th op's result;
- "loop_trips": the scan trip count (conditional_loop).
"""

import json
import re
import sys
from pathlib import Path

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/golden")
OUT = Path(__file__).with_name("reference_snapshots.json")

_BIN = {"+": "add", "-": "sub", "*": "mul", "/": "div", "<=": "le", "<": "lt", ">=": "ge", ">": "gt"}


def _offsets(text: str) -> dict:
    out = {}
    for m in re.finditer(r"device float\* (arg\d+) = arg\d+_base \+ (.+);", text):
        arg, expr = m.groups()
        terms = []
        if expr.strip() != "0":
            for t in expr.split("+"):
                tm = re.match(r"\s*\(int\)_pid\.([xyz]) \* (\d+)\s*$", t)
                if not tm:
                    raise ValueError(f"unrecognised offset term {t!r}")
                terms.append(["xyz".index(tm.group(1)), int(tm.group(2))])
        out[arg] = terms
    return out


def _block_loads(text: str) -> dict:
    """tN -> operand for `tN[_i] = argK[_i];` copy loops, with their length."""
    loads = {}
    for m in re.finditer(r"float (t\d+)\[(\d+)\];\n\s*for \(uint _i\d+ = 0; _i\d+ < \d+; \+\+_i\d+\) \{\n"
                         r"\s*t\d+\[_i\d+\] = (arg\d+)\[_i\d+\];", text):
        loads[m.group(1)] = (m.group(3), int(m.group(2)))
    return loads


def _ops(text: str, names: dict) -> list:
    ops = []
    pat_bin = re.compile(r"^\s*(t\d+)\[_i\d+\] = (\S+) (<=|>=|<|>|[-+*/]) (\S+);$")
    pat_sel = re.compile(r"^\s*(t\d+)\[_i\d+\] = (\S+) \? (\S+) : (\S+);$")

    def norm(tok: str) -> str:
        tok = re.sub(r"\[_i\d+\]$", "", tok)
        if tok in names:
            return names[tok]
        if re.match(r"^-?[0-9.e-]+f$", tok):
            return repr(float(tok[:-1]))
        raise ValueError(tok)

    for line in text.splitlines():
        m = pat_sel.match(line)
        if m:
            dst, c, a, b = m.groups()
            # select_n(pred, false_case, true_case): JAX's operand order
            ops.append(["select_n", norm(c), norm(b), norm(a)])
            names[dst] = f"e{len(ops) - 1}"
            continue
        m = pat_bin.match(line)
        if m:
            dst, lhs, op, rhs = m.groups()
            ops.append([_BIN[op], norm(lhs), norm(rhs)])
            names[dst] = f"e{len(ops) - 1}"
    return ops


def conditional_loop() -> dict:
    text = (REF / "conditional_loop.metal").read_text()
    loads = _block_loads(text)
    # t0 <- arg1 (r, the scan's const), t2 <- arg0 (y0), t4 = copy of t2: the carry
    names = {t: ("in1" if a == "arg1" else "in0") for t, (a, _) in loads.items()}
    carry = re.search(r"float (t\d+)\[64\];\n\s*for \(uint _i\d+ = 0; _i\d+ < 64; \+\+_i\d+\) \{\n"
                      r"\s*t\d+\[_i\d+\] = t\d+\[_i\d+\];", text).group(1)
    names[carry] = "carry"
    body = text[text.index("for (uint _s"):]
    body = body[: body.index("_cb")]
    trips = int(re.search(r"for \(uint _s\d+ = 0; _s\d+ < (\d+);", text).group(1))
    return {"source": "tests/golden/conditional_loop.metal", "offsets": _offsets(text), "elements": 64,
            "loop_trips": trips, "ops": _ops(body, names)}


def blocked_saxpy() -> dict:
    text = (REF / "blocked_saxpy.metal").read_text()
    loads = _block_loads(text)
    names = {t: ("in0" if a == "arg0" else "in1") for t, (a, _) in loads.items()}
    (n,) = {k for _, k in loads.values()}
    return {"source": "tests/golden/blocked_saxpy.metal", "offsets": _offsets(text), "elements": n,
            "ops": _ops(text, names)}


def copy_2d() -> dict:
    text = (REF / "copy_2d.metal").read_text()
    loads = _block_loads(text)
    ((t, (arg, n)),) = loads.items()
    store = re.search(r"(arg\d+)\[_i\d+\] = " + t + r"\[_i\d+\];", text).group(1)
    return {"source": "tests/golden/copy_2d.metal", "offsets": _offsets(text), "elements": n,
            "copy": [arg, store], "ops": []}


def main() -> None:
    data = {"conditional_loop": conditional_loop(), "blocked_saxpy": blocked_saxpy(), "copy_2d": copy_2d()}
    OUT.write_text("{\n" + ",\n".join(f' "{k}": {json.dumps(v)}' for k, v in data.items()) + "\n}\n")
    print(json.dumps(data))


if __name__ == "__main__":
    main()
