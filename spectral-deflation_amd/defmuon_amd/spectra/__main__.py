"""python -m defmuon_amd.spectra {rsvd,convergence} --dumps DIR --out DIR

rsvd         rSVD head accuracy: <out>/rsvd_accuracy.csv (spectra/rsvd_accuracy.py)
convergence  polar-factor convergence: <out>/<tag>_polar_convergence.csv per dump
             folder (tag = the folder's name) and <out>/polar_convergence_summary.csv
             (spectra/polar_convergence.py)
"""

import argparse
import csv
import os
import sys


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m defmuon_amd.spectra")
    ap.add_argument("study", choices=["rsvd", "convergence"])
    ap.add_argument("--dumps", required=True, help="a folder of dumps (rsvd) or of tag "
                    "folders of dumps (convergence)")
    ap.add_argument("--out", required=True)
    ap.add_argument("--seeds", type=int, default=20, help="sketch seeds per matrix (rsvd)")
    ap.add_argument("--tags", nargs="*", default=None)
    ap.add_argument("--iter-dtype", choices=["bf16", "fp32"], default="fp32",
                    help="precision of the polynomial iteration (convergence)")
    args = ap.parse_args(argv)
    import torch
    from defmuon_amd.spectra import accuracy as acc
    from defmuon_amd.spectra.dumps import load_matrices
    if not torch.cuda.is_available():
        print("the spectra studies run on a GPU", file=sys.stderr)
        return 1
    os.makedirs(args.out, exist_ok=True)
    log = lambda s: print(s, flush=True)
    if args.study == "rsvd":
        rows = acc.rsvd_accuracy(load_matrices(args.dumps), args.seeds, log=log)
        path = os.path.join(args.out, "rsvd_accuracy.csv")
        acc.write_rsvd_csv(rows, path)
        log(f"wrote {path}")
        return 0
    tags = args.tags or sorted(d for d in os.listdir(args.dumps)
                               if os.path.isdir(os.path.join(args.dumps, d)))
    for tag in tags:
        rows = acc.polar_convergence(load_matrices(os.path.join(args.dumps, tag)),
                                     args.iter_dtype, tag=tag, log=log)
        if rows:
            path = os.path.join(args.out, f"{tag}_polar_convergence.csv")
            acc.write_convergence_csv(rows, path)
            log(f"wrote {path}")
    merged = []
    for fn in sorted(os.listdir(args.out)):
        if fn.endswith("_polar_convergence.csv"):
            with open(os.path.join(args.out, fn)) as f:
                merged.extend(csv.DictReader(f))
    if merged:
        path = os.path.join(args.out, "polar_convergence_summary.csv")
        acc.write_convergence_csv(merged, path)
        log(f"wrote {path} ({len(merged)} rows)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
