"""Write the golden vectors of the reference CPU mixer (run in the build container only).

What this pins that nothing else does: the reference's own float32 rounding of its batched
per-token formulation, `matrix_lattice_iir` (model/mira_mixer.py:246-387), on identical seeded
inputs; and the layer stack around it -- MiraMixer's projections, control SiLU, split and
out_proj, MiraBlock's norms and feed-forward, MiraLLM's final norm with bias and tied head, and
decoding through the reference PrefixCache (`stack_*` fixtures). Stage maps, the K=1 recurrence, the stage loop and the chunk composition are pinned
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
    for arch in ("cauchy_x_hyperbolic", "expsoftplus_x_mobius"):
        out.append((f"stack_{arch}", "stack", dict(arch=arch, seed=6)))
    for arch in L.ARCH_STAGE:
        out.append((f"grad_k2m16_{arch}", "grad",
                    dict(B=2, T=45, C=5, K=2, M=16, arch=arch, mask=True, seed=7)))
    for K, M, arch in ((1, 8, "cauchy_x_mobius"), (4, 8, "expsoftplus_x_hyperbolic"),
                       (2, 64, "cauchy_x_hyperbolic"), (8, 16, "gaussian_x_identity"),
                       (2, 32, "hill_x_mobius")):
        out.append((f"grad_k{K}m{M}_{arch}", "grad",
                    dict(B=2, T=70, C=6, K=K, M=M, arch=arch, mask=False, seed=8)))
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
        elif kind == "grad":
            arrays = grad_case(torch, mixer, L, rng, p)
            y = arrays["y"]
        elif kind == "stack":
            arrays = stack_case(torch, reference_root, rng, p["arch"])
            y = arrays["llm_logits"]
        else:
            q, k, v, g = Bl.gla_inputs(rng, p["B"], p["T"], p["H"], p["dk"], p["dv"])
            S0 = (rng.standard_normal((p["B"], p["H"], p["dv"], p["dk"])) * 0.1).astype(np.float32)
            inputs = Bl.gla_as_lattice(q, k, v, g, S0)
            y, final = reference(*inputs[:7], None, inputs[7], "cauchy_x_hyperbolic")
            arrays = dict(q=q, k=k, v=v, g=g, S0=S0, y=y, final=final)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print(f"{name}: y {y.shape} max|y| {np.abs(y).max():.4g}", flush=True)


def grad_case(torch, mixer, L, rng, p):
    """Gradients of sum(dy * y) through the reference's `matrix_lattice_iir` on the CPU in
    float32 (autograd through its checkpointed per-token chunks, model/mira_mixer.py:246-387):
    what the plugin's MatrixLatticeIIR.backward must return (kernel/cuda/mira_dspv2/check.py:
    42-104 compares against exactly this). Inputs drawn as the reference harness draws them
    (check.py:52-69), from a zero state."""
    B, T, C, K, M = p["B"], p["T"], p["C"], p["K"], p["M"]
    values = L.random_inputs(rng, B, T, C, K, M)
    valid = (rng.random((B, T)) > 0.25) if p["mask"] else None
    dy = rng.standard_normal((B, T, C)).astype(np.float32)
    tensors = [torch.from_numpy(np.ascontiguousarray(v)).requires_grad_(True) for v in values]
    x, alpha, rho, gamma, write, read, beta = tensors
    y = mixer.matrix_lattice_iir(x, alpha, rho, gamma, write, read,
                                 valid=None if valid is None else torch.from_numpy(valid),
                                 raw_beta=beta, arch=p["arch"])
    (y * torch.from_numpy(dy)).sum().backward()
    names = ("x", "alpha", "rho", "gamma", "write", "read", "beta")
    arrays = {name: value for name, value in zip(names, values)}
    arrays.update({f"d{name}": tensor.grad.numpy().copy() for name, tensor in zip(names, tensors)})
    arrays.update(y=y.detach().numpy(), dy=dy, arch=np.array(p["arch"]))
    if valid is not None:
        arrays["valid"] = valid
    return arrays


STACK = dict(vocab_size=40, n_layer=2, n_embd=24, lattice_d_e=12, lattice_order=2,
             coefficient_bottleneck=6, memory_dimension=4, ffn_hidden=32)


def stack_case(torch, reference_root, rng, arch):
    """The reference's MiraMixer, MiraBlock and a 2-layer MiraLLM (model/mira_mixer.py:544-856,
    model/mira_block.py:156-205, model/mira_llm.py:20-364) on the CPU in float32, eval mode, with
    every parameter redrawn from `rng` (so the coefficient projection, the control SiLU, the FFN,
    the final norm's bias and the tied head all move the outputs). Saved: the LLM's parameters
    under their state_dict names (`p.<name>`), token ids, a padding mask, the mixer / block /
    LLM outputs, and the logits of the same ids fed as a prompt then one token at a time through
    the reference PrefixCache (`steps_logits`)."""
    llm_module = __import__("model.mira_llm", fromlist=["MiraLLM"])
    cache_module = __import__("model.prefix_cache", fromlist=["PrefixCache"])
    modulus, argument = arch.split("_x_")
    torch.manual_seed(0)
    model = llm_module.MiraLLM(lattice_modulus_map=modulus, lattice_argument_map=argument,
                               **STACK).eval()
    with torch.no_grad():
        for name, parameter in model.named_parameters():
            scale = 0.1 if name.endswith(("rn1.weight", "rn2.weight", "lnf.weight")) else 0.3
            value = rng.standard_normal(tuple(parameter.shape)) * scale
            if name.endswith(("rn1.weight", "rn2.weight", "lnf.weight")):
                value = value + 1.0
            parameter.copy_(torch.from_numpy(value.astype(np.float32)))
    B, T, prompt = 2, 11, 6
    ids = rng.integers(0, STACK["vocab_size"], size=(B, T))
    mask = np.ones((B, T), dtype=bool)
    mask[0, :2] = False                       # left padding on the first row
    mask[1, 7] = False                        # and one masked token inside the second
    d = STACK["n_embd"]
    hidden = rng.standard_normal((B, T, d)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    with torch.no_grad():
        block = model.blocks[0]
        mixer_out = block.mixer(block.rn1(t(hidden)), t(mask))
        block_out = block(t(hidden), t(mask))
        logits = model(t(ids), attention_mask=t(mask)).logits
        cache = cache_module.PrefixCache(STACK["n_layer"], budget=0)
        steps = [model(t(ids[:, :prompt]), cache=cache).logits]
        for i in range(prompt, T):
            steps.append(model(t(ids[:, i:i + 1]), cache=cache).logits)
        steps_logits = torch.cat(steps, dim=1)
    arrays = {f"p.{name}": value.detach().numpy().copy()
              for name, value in model.state_dict().items()}
    arrays.update(ids=ids.astype(np.int64), mask=mask, hidden=hidden,
                  mixer_out=mixer_out.numpy(), block_out=block_out.numpy(),
                  llm_logits=logits.numpy(), steps_logits=steps_logits.numpy(), prompt=prompt,
                  arch=np.array(arch))
    return arrays


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", default="/root/reference")
    run(os.path.abspath(parser.parse_args().reference))
