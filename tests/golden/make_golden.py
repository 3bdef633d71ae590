"""Write the golden fixtures of the pair-stack path (run from the repo root:
``python tests/golden/make_golden.py``).

The reference holds no golden vectors for this path, so the fixtures are made
here: seeded inputs and weights, and expected outputs computed by the oracle
in float64.  Each expected output is first checked against the independent
float64 scalar-loop formulation in ``tests/brute_force.py`` (a dropped term
or swapped index in either would disagree), and only then stored.  Triangle
attention with padded tokens is stored as the oracle's float32 result: the
reference's -1e9 mask term makes a fully masked row uniform in float32 but
not in float64; its rows that keep a key are checked against float64, its
padded rows against a direct mean-of-V computation.  Shapes
are chosen inside what the HIP kernels take (c in {64, 128}, head dim 32) so
that the same files feed the GPU parity tests; ragged token counts and
padded (fully masked) tokens are included.

Each ``.npz`` holds plain arrays only (load with ``allow_pickle=False``):
inputs (``z``, ``mask``, ``s``, ``x``), parameters under ``p.<name>`` in the
reference's parameter names, float32, and ``expected*`` in float32.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.dirname(HERE)]

import brute_force as bf  # noqa: E402
from helpers import params_of, seeded, token_pair_mask  # noqa: E402
from oracle import reference as ref  # noqa: E402
from opendde_amd.pairformer import PairformerBlock, Transition  # noqa: E402
from opendde_amd.triangular import (TriangleAttention, TriangleMultiplicationIncoming,  # noqa: E402
                                    TriangleMultiplicationOutgoing)

STD = 0.1


def _f64(p):
    return {k: v.double() for k, v in p.items()}


def _save(name, arrays, params):
    out = {k: np.ascontiguousarray(v.detach().cpu().float().numpy()) for k, v in arrays.items()}
    out.update({f"p.{k}": np.ascontiguousarray(v.float().numpy()) for k, v in params.items()})
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def _check(expected, brute, what, tol=1e-9):
    err = float(np.abs(expected.double().numpy() - brute).max())
    assert err < tol, f"{what}: oracle vs brute force {err:.3e}"


def _masked_rows_uniform(z, p, h, starting):
    """Rows whose token is padded: every logit carries -1e9, which absorbs
    q.k + bias in the reference's float32 arithmetic, so the softmax is
    uniform and the update is W_o(sigmoid(g) * mean_k v).  Computed directly
    in float64 (no softmax)."""
    zz = z.double() if starting else z.double().transpose(0, 1)
    x = torch.nn.functional.layer_norm(zz, (zz.shape[-1],), p["layer_norm.weight"].double(),
                                       p["layer_norm.bias"].double(), 1e-5)
    v = (x @ p["mha.linear_v.weight"].double().t()).view(*x.shape[:2], h, 32)
    gt = torch.sigmoid(x @ p["mha.linear_g.weight"].double().t()).view(*x.shape[:2], h, 32)
    o = gt * v.mean(dim=1, keepdim=True)
    upd = o.reshape(*x.shape[:2], h * 32) @ p["mha.linear_o.weight"].double().t()
    return upd if starting else upd.transpose(0, 1)


def triangle_attention(starting: bool):
    n, c, h = 20, 64, 2
    mod = seeded(TriangleAttention(c, 32, h, starting=starting), 11 if starting else 12, STD)
    g = torch.Generator().manual_seed(13)
    z = torch.randn(n, n, c, generator=g)
    t = torch.ones(n)
    t[torch.randperm(n, generator=torch.Generator().manual_seed(5))[:3]] = 0
    mask = t[:, None] * t[None, :]
    p = params_of(mod)
    exp64 = ref.triangle_attention(z.double(), mask.double(), _f64(p), h, starting=starting)
    _check(exp64, bf.triangle_attention(z, mask, p, h, starting=starting), "triangle attention")
    # the stored result is the reference's float32 arithmetic
    exp = ref.triangle_attention(z, mask, p, h, starting=starting)
    keep = t.bool()
    rows = (lambda a: a[keep]) if starting else (lambda a: a[:, keep])
    prow = (lambda a: a[~keep]) if starting else (lambda a: a[:, ~keep])
    assert float((rows(exp).double() - rows(exp64)).abs().max()) < 1e-5
    uni = _masked_rows_uniform(z, p, h, starting)
    assert float((prow(exp).double() - prow(uni)).abs().max()) < 1e-5
    _save(f"triatt_{'start' if starting else 'end'}_n{n}_c{c}_h{h}",
          {"z": z, "mask": mask, "expected": exp}, p)


def triangle_multiplication(outgoing: bool):
    n, c, ch = 19, 64, 64
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(c, ch), 21 if outgoing else 22, STD)
    g = torch.Generator().manual_seed(23)
    z = torch.randn(n, n, c, generator=g)
    mask = token_pair_mask(n, 2, seed=6, random=True)
    p = params_of(mod)
    exp = ref.triangle_multiplication(z.double(), mask.double(), _f64(p), outgoing)
    _check(exp, bf.triangle_multiplication(z, mask, p, outgoing), "triangle multiplication")
    _save(f"trimul_{'out' if outgoing else 'in'}_n{n}_c{c}_ch{ch}",
          {"z": z, "mask": mask, "expected": exp}, p)


def transition():
    rows, c = 150, 64
    mod = seeded(Transition(c, 4), 31, STD)
    x = torch.randn(rows, c, generator=torch.Generator().manual_seed(32))
    p = params_of(mod)
    exp = ref.transition(x.double(), _f64(p))
    _check(exp, bf.transition(x, p), "transition")
    _save(f"transition_rows{rows}_c{c}", {"x": x, "expected": exp}, p)


def block():
    n, cz, cs, heads = 14, 64, 64, 16
    mod = seeded(PairformerBlock(n_heads=heads, c_z=cz, c_s=cs, c_hidden_mul=64,
                                 c_hidden_pair_att=32, no_heads_pair=2), 41, 0.05)
    g = torch.Generator().manual_seed(42)
    z = torch.randn(n, n, cz, generator=g)
    s = torch.randn(n, cs, generator=g)
    # unpadded: with padded tokens the block's float32 and float64 results
    # part on the fully masked attention rows (covered by the module fixtures)
    mask = token_pair_mask(n, 0)
    p = params_of(mod)
    se, ze = ref.pairformer_block(s.double(), z.double(), mask.double(), _f64(p),
                                  no_heads_pair=2, n_heads=heads)
    bs, bz = bf.pairformer_block(s, z, mask, p, 2, heads)
    _check(ze, bz, "block z")
    _check(se, bs, "block s")
    _save(f"block_n{n}_cz{cz}_cs{cs}", {"z": z, "s": s, "mask": mask, "expected_z": ze,
                                        "expected_s": se}, p)


if __name__ == "__main__":
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    triangle_attention(True)
    triangle_attention(False)
    triangle_multiplication(True)
    triangle_multiplication(False)
    transition()
    block()
