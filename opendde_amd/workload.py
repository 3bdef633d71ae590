"""Synthetic workloads for the Pairformer pair stack (seeded inputs + weights).

Conventions (fixed here so that tests, smoke and bench draw identical data):

* generator: ``torch.Generator('cpu').manual_seed(seed)``; draw order is the
  pair tensor z, then the single tensor s, then the token mask, then the
  parameters in ``sorted(named_parameters())`` order; everything is drawn on
  the CPU in float32 and moved afterwards;
* Linear weights (and biases) ~ N(0, std^2), std = 0.02;
* LayerNorm weight = 1 + N(0, std^2), LayerNorm bias ~ N(0, std^2).  (Pure
  N(0, 0.02) LayerNorm gains would shrink every activation to ~1e-4 and make
  absolute tolerances vacuous.)
* token mask t[N]: ones, with ``n_pad`` tokens set to 0 (either the last
  ``n_pad`` or a seeded random subset); pair mask = t[:, None] * t[None, :].
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Iterable, Optional, Tuple

import torch

STD = 0.02


def generator(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(int(seed))


def _is_ln_param(name: str) -> bool:
    leaf = name.rsplit(".", 2)
    mod = leaf[-2] if len(leaf) >= 2 else ""
    return "layer_norm" in mod or "layernorm" in mod


def param_values(specs: Iterable[Tuple[str, Tuple[int, ...]]], gen: torch.Generator,
                 std: float = STD) -> Dict[str, torch.Tensor]:
    """Draw values for (name, shape) specs, in sorted-name order."""
    out = {}
    for name, shape in sorted(specs):
        t = torch.randn(shape, generator=gen, dtype=torch.float32) * std
        if _is_ln_param(name) and name.endswith(".weight"):
            t = t + 1.0
        out[name] = t
    return out


def init_module_(module: torch.nn.Module, gen: torch.Generator, std: float = STD) -> None:
    """Overwrite every parameter of ``module`` with the workload convention."""
    specs = [(n, tuple(p.shape)) for n, p in module.named_parameters()]
    vals = param_values(specs, gen, std)
    with torch.no_grad():
        for n, p in module.named_parameters():
            p.copy_(vals[n].to(p.device, p.dtype))


def token_mask(n: int, n_pad: int, gen: Optional[torch.Generator] = None,
               random: bool = False) -> torch.Tensor:
    t = torch.ones(n, dtype=torch.float32)
    if n_pad > 0:
        if random:
            idx = torch.randperm(n, generator=gen)[:n_pad]
            t[idx] = 0.0
        else:
            t[n - n_pad:] = 0.0
    return t


def pair_mask(t: torch.Tensor) -> torch.Tensor:
    return t[:, None] * t[None, :]


# --- parameter name/shape specs with the reference's names --------------------


def triatt_specs(c: int, h: int, d: int = 32, prefix: str = ""):
    hd = h * d
    return [
        (prefix + "layer_norm.weight", (c,)), (prefix + "layer_norm.bias", (c,)),
        (prefix + "linear.weight", (h, c)),
        (prefix + "mha.linear_q.weight", (hd, c)), (prefix + "mha.linear_k.weight", (hd, c)),
        (prefix + "mha.linear_v.weight", (hd, c)), (prefix + "mha.linear_o.weight", (c, hd)),
        (prefix + "mha.linear_g.weight", (hd, c)),
    ]


def trimul_specs(c: int, ch: int, prefix: str = ""):
    return [
        (prefix + "layer_norm_in.weight", (c,)), (prefix + "layer_norm_in.bias", (c,)),
        (prefix + "layer_norm_out.weight", (ch,)), (prefix + "layer_norm_out.bias", (ch,)),
        (prefix + "linear_a_p.weight", (ch, c)), (prefix + "linear_a_g.weight", (ch, c)),
        (prefix + "linear_b_p.weight", (ch, c)), (prefix + "linear_b_g.weight", (ch, c)),
        (prefix + "linear_z.weight", (c, ch)), (prefix + "linear_g.weight", (c, c)),
    ]


def transition_specs(c: int, n: int = 4, prefix: str = ""):
    return [
        (prefix + "layernorm1.weight", (c,)), (prefix + "layernorm1.bias", (c,)),
        (prefix + "linear_no_bias_a.weight", (n * c, c)),
        (prefix + "linear_no_bias_b.weight", (n * c, c)),
        (prefix + "linear_no_bias.weight", (c, n * c)),
    ]


def opm_specs(c_m: int, c: int, c_z: int, prefix: str = ""):
    """OuterProductMean(c_m, c_z, c_hidden=c) parameters (the reference's
    OpenfoldLinear defaults: linear_1 / linear_2 built with bias=False,
    linear_out with a bias; triangular/layers.py:518-521)."""
    return [
        (prefix + "layer_norm.weight", (c_m,)), (prefix + "layer_norm.bias", (c_m,)),
        (prefix + "linear_1.weight", (c, c_m)),
        (prefix + "linear_2.weight", (c, c_m)),
        (prefix + "linear_out.weight", (c_z, c * c)), (prefix + "linear_out.bias", (c_z,)),
    ]


def apb_specs(c_s: int, c_z: int, n_heads: int, prefix: str = ""):
    return [
        (prefix + "layernorm_a.weight", (c_s,)), (prefix + "layernorm_a.bias", (c_s,)),
        (prefix + "attention.linear_q.weight", (c_s, c_s)),
        (prefix + "attention.linear_q.bias", (c_s,)),
        (prefix + "attention.linear_k.weight", (c_s, c_s)),
        (prefix + "attention.linear_v.weight", (c_s, c_s)),
        (prefix + "attention.linear_o.weight", (c_s, c_s)),
        (prefix + "attention.linear_g.weight", (c_s, c_s)),
        (prefix + "layernorm_z.weight", (c_z,)), (prefix + "layernorm_z.bias", (c_z,)),
        (prefix + "linear_nobias_z.weight", (n_heads, c_z)),
    ]


def block_specs(c_z: int = 128, c_s: int = 384, h: int = 4, d: int = 32, ch: int = 128,
                n_heads: int = 16, prefix: str = ""):
    s = []
    s += trimul_specs(c_z, ch, prefix + "tri_mul_out.")
    s += trimul_specs(c_z, ch, prefix + "tri_mul_in.")
    s += triatt_specs(c_z, h, d, prefix + "tri_att_start.")
    s += triatt_specs(c_z, h, d, prefix + "tri_att_end.")
    s += transition_specs(c_z, 4, prefix + "pair_transition.")
    if c_s > 0:
        s += apb_specs(c_s, c_z, n_heads, prefix + "attention_pair_bias.")
        s += transition_specs(c_s, 4, prefix + "single_transition.")
    return s


def stack_specs(n_blocks: int, **kw):
    s = []
    for b in range(n_blocks):
        s += block_specs(prefix=f"blocks.{b}.", **kw)
    return s


@dataclass(frozen=True)
class PairConfig:
    """One named workload: a pair tensor of N tokens and its member dims."""

    name: str
    n: int
    c_z: int = 128
    c_s: int = 384
    heads: int = 4
    head_dim: int = 32
    c_hidden_mul: int = 128
    n_heads_single: int = 16
    n_blocks: int = 1
    n_pad: int = 0
    random_pad: bool = False
    seed: int = 0


# The five workloads the path is specified on.
BLOCK_N128 = PairConfig("pairformer_block_n128_fp32", 128, seed=0)
TRIATT_N384 = PairConfig("triangle_attention_start_n384_bf16", 384, c_s=0,
                         n_pad=38, seed=1)
TRIMUL_N768 = PairConfig("triangle_multiplication_n768_bf16", 768, c_s=0, seed=2)
TRUNK_N1024 = PairConfig("pairformer_trunk_48x_n1024_bf16", 1024, n_blocks=48,
                         n_pad=51, random_pad=True, seed=3)
STRESS_N2048 = PairConfig("pairformer_4x_n2048_bf16", 2048, n_blocks=4, seed=4)


def make_inputs(cfg: PairConfig, with_s: Optional[bool] = None):
    """Draw (z, s, pair_mask, gen) on the CPU in float32; the returned
    generator continues with the parameter draws."""
    gen = generator(cfg.seed)
    z = torch.randn((cfg.n, cfg.n, cfg.c_z), generator=gen, dtype=torch.float32)
    want_s = (cfg.c_s > 0) if with_s is None else with_s
    s = torch.randn((cfg.n, cfg.c_s), generator=gen, dtype=torch.float32) if want_s else None
    t = token_mask(cfg.n, cfg.n_pad, gen, cfg.random_pad)
    return z, s, pair_mask(t), gen
