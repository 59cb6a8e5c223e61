"""Write golden vectors for the polar-factor path from the reference itself.

Run in the build container only (the reference tree is not present on the GPU box):

    python tests/golden/make_golden.py [/path/to/reference]

It imports the reference's hot-path modules (defmuon/optim/{muon,polar_express,
deflation_batched}.py) on the CPU and records their outputs on small seeded inputs
into tests/golden/*.npz.  The fixtures hold data only: inputs, injected sketches and
the reference's outputs.  Two rounding modes are recorded for the bf16 chains:

    eager     TorchDynamo disabled (every op rounds to bf16)
    compiled  torch.compile with inductor on the CPU, as the reference runs them

The deflation front-end (batched_rmfro_clip) is never compiled by the reference,
so one eager fp32 record covers it.
"""

import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))


def _bits(t):
    """bf16 tensor -> uint16 numpy array of its bit patterns."""
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _inputs():
    import torch
    sys.path.insert(0, os.path.join(REPO, "spectral-deflation_amd"))
    from defmuon_amd import synthetic as S
    ins = {}
    # front-end: B=2 tall (192, 96) spiked matrices, k = 2 by design, r = 6, kw = 3
    A = torch.stack([S.spiked_matrix(192, 96, seed=11 + i, n_spikes=2, hi=50.0, lo=20.0)
                     for i in range(2)])
    g = torch.Generator().manual_seed(7)
    ins["clip_A"] = A
    ins["clip_Omega"] = torch.randn(2, 96, 6, generator=g)
    # front-end with the gate firing on matrix 0 (k = 1) and declining on matrix 1
    # (pure bulk); m = 80 gives r = 4, kw = 2
    A2 = torch.stack([S.spiked_matrix(160, 80, seed=21, n_spikes=1, hi=80.0, lo=80.0),
                      S.spiked_matrix(160, 80, seed=22, n_spikes=0)])
    ins["clip2_A"] = A2
    ins["clip2_Omega"] = torch.randn(2, 80, 4, generator=g)
    # plain arms: wide, tall and a W_QKV-like (3, d, d) stack
    ins["wide_G"] = torch.randn(96, 256, generator=g)
    ins["tall_G"] = torch.randn(256, 96, generator=g)
    ins["qkv_G"] = torch.randn(3, 64, 64, generator=g)
    return ins


def _run(mode, ref):
    """Child process: import the reference in `mode` and dump its outputs."""
    import torch
    os.environ["DEFMUON_COMPILE_DEFL_ITER"] = "1" if mode == "compiled" else "0"
    sys.path.insert(0, ref)
    from defmuon.optim import deflation_batched as DB
    from defmuon.optim import muon as MU
    from defmuon.optim import polar_express as PE
    torch.manual_seed(0)
    ins = _inputs()
    out = {}
    for key in ("clip", "clip2"):
        A, Om = ins[f"{key}_A"], ins[f"{key}_Omega"]
        U, s, V = DB._rsvd_b(A, Om, DB.RSVD_NITER)
        X0f, k, d = DB.batched_rmfro_clip(A, Omega=Om, pad=DB.DIVISOR_PAD)
        X0, _, _ = DB.batched_rmfro_clip(A, Omega=Om, pad=DB.DIVISOR_PAD,
                                         out_dtype=torch.bfloat16)
        X0pe, kpe, dpe = DB.batched_rmfro_clip(A, Omega=Om, pad=DB.DeflatedPEPolar.PAD,
                                               out_dtype=torch.bfloat16)
        out[f"{key}_s"] = s.numpy()
        out[f"{key}_head_proj"] = (U[..., :2] @ V[..., :2].mT).numpy()
        out[f"{key}_X0f32"] = X0f.numpy()
        out[f"{key}_X0"] = _bits(X0)
        out[f"{key}_k"] = k.numpy()
        out[f"{key}_d"] = d.numpy()
        out[f"{key}_X0pe"] = _bits(X0pe)
        out[f"{key}_kpe"] = kpe.numpy()
        ns = DB.DeflatedNSPolar()._iterate(X0, 5)
        pe = DB.DeflatedPEPolar()._iterate(X0pe, 5)
        out[f"{key}_iter_ns"] = _bits(ns)
        out[f"{key}_iter_pe"] = _bits(pe)
    Q = DB._orth_b(ins["clip_A"] @ ins["clip_Omega"])
    out["orth_Q"] = Q.numpy()
    for name in ("wide_G", "tall_G", "qkv_G"):
        out[f"{name}_ns5"] = _bits(MU.zeropower_via_newtonschulz5(ins[name], 5))
        out[f"{name}_pe"] = _bits(PE.PolarExpress(ins[name], 5))
    np.savez_compressed(os.path.join(HERE, f"ref_{mode}.npz"), **out)
    print(f"wrote ref_{mode}.npz ({len(out)} arrays)")


def main():
    if len(sys.argv) > 2 and sys.argv[1] == "--child":
        _run(sys.argv[2], sys.argv[3])
        return
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ins = _inputs()
    np.savez_compressed(os.path.join(HERE, "inputs.npz"),
                        **{k: v.numpy() for k, v in ins.items()})
    print("wrote inputs.npz")
    for mode in ("eager", "compiled"):
        env = dict(os.environ)
        if mode == "eager":
            env["TORCHDYNAMO_DISABLE"] = "1"
        else:
            env.pop("TORCHDYNAMO_DISABLE", None)
        subprocess.run([sys.executable, os.path.abspath(__file__), "--child", mode, ref],
                       check=True, env=env, cwd=REPO)


if __name__ == "__main__":
    main()
