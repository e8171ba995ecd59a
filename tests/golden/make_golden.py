"""Write the golden vectors of the reference CPU mixer (run in the build container only).

What this pins that nothing else does: the reference's own float32 rounding of its batched
per-token formulation, `matrix_lattice_iir` (model/mira_mixer.py:246-387), on identical seeded
inputs. Stage maps, the K=1 recurrence, the stage loop and the chunk composition are pinned
independently by closed forms and invariants in tests/test_oracle.py; these vectors pin the
literal "max abs error against the reference's CPU mixer" criterion.

The reference is imported from REFERENCE (default /root/reference) in this container; neither
it nor any of its bytecode is written into the repository. Only inputs and outputs are saved,
as small float32 .npz fixtures next to this script.

    python tests/golden/make_golden.py [--reference /root/reference]
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def cases():
    """(name, kind, parameters): the fixture set, each small enough to run on the CPU in seconds."""
    sys.path.insert(0, ROOT)
    from oracle import lattice as L  # noqa: E402

    out = []
    for arch in L.ARCH_STAGE:
        out.append((f"k2m16_{arch}", "lattice",
                    dict(B=2, T=37, C=5, K=2, M=16, arch=arch, mask=True, state=True, seed=1)))
    for K, M in ((1, 1), (1, 8), (4, 8), (8, 4), (2, 64), (1, 128)):
        out.append((f"k{K}m{M}_cauchy_x_hyperbolic", "lattice",
                    dict(B=2, T=70, C=6, K=K, M=M, arch="cauchy_x_hyperbolic", mask=False,
                         state=True, seed=2)))
    out.append(("k2m16_long_unmasked", "lattice",
                dict(B=1, T=300, C=8, K=2, M=16, arch="cauchy_x_hyperbolic", mask=False,
                     state=False, seed=3, beta_bias=0.0, alpha_bias=0.5)))
    out.append(("diag_cfg1_reduced", "diag", dict(B=1, T=512, D=32, seed=4)))
    out.append(("gla_cfg3_reduced", "gla", dict(B=1, T=96, H=2, dk=16, dv=16, seed=5)))
    return out


def run(reference_root):
    sys.path.insert(0, ROOT)
    from oracle import lattice as L, baseline as Bl  # noqa: E402

    sys.path.insert(0, reference_root)
    os.chdir(reference_root)
    import torch  # noqa: E402
    mixer = __import__("model.mira_mixer", fromlist=["matrix_lattice_iir"])
    torch.set_num_threads(1)

    def reference(x, alpha, rho, gamma, write, read, beta, valid, state, arch):
        t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
        with torch.no_grad():
            y, final = mixer.matrix_lattice_iir(
                t(x), t(alpha), t(rho), t(gamma), t(write), t(read),
                valid=None if valid is None else torch.from_numpy(valid),
                raw_beta=t(beta), state=t(state), return_state=True, arch=arch)
        return y.numpy(), final.numpy()

    for name, kind, p in cases():
        rng = np.random.default_rng(p["seed"])
        if kind == "lattice":
            B, T, C, K, M = p["B"], p["T"], p["C"], p["K"], p["M"]
            x, alpha, rho, gamma, write, read, beta = L.random_inputs(
                rng, B, T, C, K, M, alpha_bias=p.get("alpha_bias", 0.0),
                beta_bias=p.get("beta_bias", 0.0))
            valid = (rng.random((B, T)) > 0.25) if p["mask"] else None
            state = ((rng.standard_normal((B, K, C, M)) * 0.1).astype(np.float32)
                     if p["state"] else None)
            y, final = reference(x, alpha, rho, gamma, write, read, beta, valid, state, p["arch"])
            arrays = dict(x=x, alpha=alpha, rho=rho, gamma=gamma, write=write, read=read,
                          beta=beta, y=y, final=final)
            if valid is not None:
                arrays["valid"] = valid
            if state is not None:
                arrays["state"] = state
            arrays["arch"] = np.array(p["arch"])
        elif kind == "diag":
            x, a, w, bias, _ = Bl.diag_inputs(rng, p["B"], p["T"], p["D"])
            h0 = (rng.standard_normal((p["B"], p["D"])) * 0.1).astype(np.float32)
            u = Bl.causal_conv(x, w, bias, dtype=np.float32).astype(np.float32)
            inputs = Bl.diag_as_lattice(u, a, h0)
            y, final = reference(*inputs[:7], None, inputs[7], "cauchy_x_hyperbolic")
            arrays = dict(x=x, a=a, w=w, bias=bias, h0=h0, u=u, y=y, final=final)
        else:
            q, k, v, g = Bl.gla_inputs(rng, p["B"], p["T"], p["H"], p["dk"], p["dv"])
            S0 = (rng.standard_normal((p["B"], p["H"], p["dv"], p["dk"])) * 0.1).astype(np.float32)
            inputs = Bl.gla_as_lattice(q, k, v, g, S0)
            y, final = reference(*inputs[:7], None, inputs[7], "cauchy_x_hyperbolic")
            arrays = dict(q=q, k=k, v=v, g=g, S0=S0, y=y, final=final)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print(f"{name}: y {y.shape} max|y| {np.abs(y).max():.4g}", flush=True)


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", default="/root/reference")
    run(os.path.abspath(parser.parse_args().reference))
