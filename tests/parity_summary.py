"""Tabulate the parity margins a GPU test run recorded (tests/parity.py writes one
JSON line per check to $DMH_PARITY_LOG):

    DMH_PARITY_LOG=parity.jsonl python -m pytest tests -m gpu
    python tests/parity_summary.py parity.jsonl > summary.md

Polar factors: per group of checks (the tag without its matrix index), the worst
|relerr(gpu) - relerr(oracle)|, relative orthogonality-residual difference and
direct difference ||gpu - oracle||_F / ||oracle||_F against their tolerances.
Front-end: the worst relative singular-value, head-subspace, divisor and entry
differences.  Convergence study: per iteration dtype and method, the largest difference
of a relative-error curve point from the oracle's."""

import json
import re
import sys
from collections import OrderedDict

_HERE = __import__("os").path.dirname(__import__("os").path.abspath(__file__))
sys.path[:0] = [_HERE, __import__("os").path.dirname(_HERE)]
from parity import DIRECT_TOL, ORTH_TOL, POLAR_TOL  # noqa: E402


def main(path):
    polar, front, conv = OrderedDict(), OrderedDict(), OrderedDict()
    for line in open(path):
        r = json.loads(line)
        if r["kind"] == "convergence":
            words = r["tag"].split(" ")   # "<dtype> <step> <matrix> <method>"
            dtype, method = words[0], words[-1]
            g = conv.setdefault((dtype, method), dict(n=0, diff=0.0))
            g["n"] += 1
            g["diff"] = max(g["diff"], r["max_curve_diff"])
        elif r["kind"] == "polar":
            key = re.sub(r"(\s*#\d+|\[\d+\])$", "", r["tag"])
            g = polar.setdefault(key, dict(n=0, drel=0.0, dorth=0.0, direct=0.0, relerr=0.0))
            g["n"] += 1
            g["drel"] = max(g["drel"], abs(r["relerr"] - r["relerr_oracle"]))
            g["dorth"] = max(g["dorth"], abs(r["orth"] - r["orth_oracle"]) / r["orth_oracle"])
            g["direct"] = max(g["direct"], r["direct"])
            g["relerr"] = max(g["relerr"], r["relerr"])
        else:
            g = front.setdefault(r["tag"], {})
            for k, v in r.items():
                if k not in ("kind", "tag"):
                    g[k] = max(g.get(k, 0.0), v)
    print("| polar factors (checks) | max relerr vs exact | max abs(d relerr) "
          f"(tol {POLAR_TOL:g}) | max rel d orth (tol {ORTH_TOL:g}) | max direct "
          f"(tol {DIRECT_TOL:g}) |")
    print("|---|---|---|---|---|")
    for key, g in polar.items():
        print(f"| {key} ({g['n']}) | {g['relerr']:.4f} | {g['drel']:.2e} | {g['dorth']:.2e} "
              f"| {g['direct']:.2e} |")
    if front:
        print()
        print("| front-end check | max rel s err | head subspace | max rel d err | entry X0 |")
        print("|---|---|---|---|---|")
        for key, g in front.items():
            f = lambda k: f"{g[k]:.2e}" if k in g else "-"
            print(f"| {key} | {f('s')} | {f('head')} | {f('d')} | {f('x0')} |")
    if conv:
        print()
        print("| convergence curves (iteration dtype, method) | curves | max point difference "
              "from the oracle (tol: bf16 2e-2, fp32 1e-5) |")
        print("|---|---|---|")
        for (dtype, method), g in conv.items():
            print(f"| {dtype} {method} | {g['n']} | {g['diff']:.2e} |")


if __name__ == "__main__":
    main(sys.argv[1])
