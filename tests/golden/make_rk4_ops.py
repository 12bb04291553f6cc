"""Extract the RK4 Lotka-Volterra step's op sequence from the reference's
golden Metal text into a JSON fixture (run where /root/reference exists).

Source: tests/golden/rk4_lotka_volterra.metal:55-293 of the reference (the
blessed emitter output for examples/01's kernel with DT=0.01, 500 steps).
Each loop-body assignment `tN[..] = A op B;` becomes [op, A, B] with operands
normalised to: the consts "a","b","c","d", the carries "x","y", a literal
float string, or "e<k>" for the k-th body result.
"""

import json
import re
import sys
from pathlib import Path

SRC = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/golden/rk4_lotka_volterra.metal")
OUT = Path(__file__).with_name("rk4_lotka_volterra_ops.json")


def main() -> None:
    text = SRC.read_text().splitlines()
    names = {"t0": "a", "t2": "b", "t4": "c", "t6": "d", "t12": "x", "t14": "y"}
    ops = []
    in_loop = False
    pat = re.compile(r"^\s*(t\d+)\[_i\d+\] = (\S+) ([-+*/]) (\S+);$")
    for line in text:
        if "for (uint _s" in line:
            in_loop = True
            continue
        if in_loop and "_cb" in line:
            break
        m = pat.match(line)
        if not (in_loop and m):
            continue
        dst, lhs, op, rhs = m.groups()

        def norm(tok: str) -> str:
            tok = tok.replace("[0]", "")
            if tok in names:
                return names[tok]
            if tok.endswith("f") and re.match(r"^[0-9.e-]+f$", tok):
                return tok[:-1]
            raise ValueError(tok)

        ops.append([{"+": "add", "-": "sub", "*": "mul", "/": "div"}[op], norm(lhs), norm(rhs)])
        names[dst] = f"e{len(ops) - 1}"
    OUT.write_text(json.dumps({"source": "tests/golden/rk4_lotka_volterra.metal:55-293", "dt": 0.01, "ops": ops}, indent=0))
    print(f"{len(ops)} ops -> {OUT}")


if __name__ == "__main__":
    main()
