"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the float64 oracle after checking it against the float64 scalar loops).

CPU: the oracle and the torch path of the drop-in modules reproduce them.
GPU: the HIP path reproduces them, fp32 compute to max-abs 1e-4 and bf16
compute to the bf16 tier.
"""

import os

import numpy as np
import pytest
import torch

from helpers import assert_bf16, assert_fp32, say
from oracle import reference as ref
from opendde_amd.pairformer import PairformerBlock, Transition
from opendde_amd.triangular import (TriangleAttention, TriangleMultiplicationIncoming,
                                    TriangleMultiplicationOutgoing)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        arrays = {k: torch.from_numpy(f[k].copy()) for k in f.files}
    params = {k[2:]: v for k, v in arrays.items() if k.startswith("p.")}
    data = {k: v for k, v in arrays.items() if not k.startswith("p.")}
    return data, params


def module_for(name):
    if name.startswith("triatt"):
        return TriangleAttention(64, 32, 2, starting="start" in name)
    if name.startswith("trimul"):
        cls = TriangleMultiplicationOutgoing if "_out_" in name else TriangleMultiplicationIncoming
        return cls(64, 64)
    if name.startswith("transition"):
        return Transition(64, 4)
    return PairformerBlock(n_heads=16, c_z=64, c_s=64, c_hidden_mul=64, c_hidden_pair_att=32,
                           no_heads_pair=2)


def loaded(name):
    data, params = load(name)
    mod = module_for(name)
    mod.load_state_dict(params, strict=True)
    return mod.eval(), data, params


MODULE_FIXTURES = ["triatt_start_n20_c64_h2", "triatt_end_n20_c64_h2",
                   "trimul_out_n19_c64_ch64", "trimul_in_n19_c64_ch64"]


def test_fixture_files_present():
    names = sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz"))
    assert names == sorted(MODULE_FIXTURES + ["transition_rows150_c64", "block_n14_cz64_cs64"])


@pytest.mark.parametrize("name", MODULE_FIXTURES)
def test_oracle_and_torch_path_reproduce_module_fixtures(name):
    mod, d, p = loaded(name)
    if name.startswith("triatt"):
        o = ref.triangle_attention(d["z"], d["mask"], p, 2, starting="start" in name)
        t = mod(d["z"], d["mask"], triangle_attention="torch")
    else:
        o = ref.triangle_multiplication(d["z"], d["mask"], p, "_out_" in name)
        t = mod(d["z"], d["mask"], triangle_multiplicative="torch")
    torch.testing.assert_close(o, d["expected"], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(t, d["expected"], atol=1e-5, rtol=1e-5)


def test_oracle_reproduces_transition_and_block_fixtures():
    _, d, p = loaded("transition_rows150_c64")
    torch.testing.assert_close(ref.transition(d["x"], p), d["expected"], atol=1e-5, rtol=1e-5)
    mod, d, p = loaded("block_n14_cz64_cs64")
    s, z = ref.pairformer_block(d["s"], d["z"], d["mask"], p, no_heads_pair=2, n_heads=16)
    torch.testing.assert_close(z, d["expected_z"], atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(s, d["expected_s"], atol=1e-4, rtol=1e-4)
    with torch.no_grad():
        s2, z2 = mod(d["s"], d["z"].clone(), d["mask"])
    torch.testing.assert_close(z2, d["expected_z"], atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(s2, d["expected_s"], atol=1e-4, rtol=1e-4)


# --------------------------------------------------------------------- GPU


@pytest.mark.gpu
@pytest.mark.parametrize("name", MODULE_FIXTURES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hip_reproduces_module_fixtures(name, dtype):
    say(f"[gpu] golden {name} {dtype}")
    mod, d, _ = loaded(name)
    mod = mod.cuda()
    z = d["z"].cuda().to(dtype)
    mask = d["mask"].cuda()
    if name.startswith("triatt"):
        got = mod(z, mask, triangle_attention="hip")
    else:
        got = mod(z, mask, triangle_multiplicative="hip")
    if dtype == torch.float32:
        assert_fp32(got, d["expected"], f"golden {name}")
    else:
        # the fixture's input rounded to bf16 is what the kernel sees; the
        # fp32 oracle on that input is the reference for the bf16 tier
        mod_cpu, _, p = loaded(name)
        zb = d["z"].to(dtype).float()
        if name.startswith("triatt"):
            exp = ref.triangle_attention(zb, d["mask"], p, 2, starting="start" in name)
        else:
            exp = ref.triangle_multiplication(zb, d["mask"], p, "_out_" in name)
        assert_bf16(got, exp, f"golden {name} bf16")


@pytest.mark.gpu
def test_hip_reproduces_transition_fixture():
    say("[gpu] golden transition")
    mod, d, _ = loaded("transition_rows150_c64")
    mod = mod.cuda()
    got = mod.hip_apply(d["x"].cuda().to(torch.bfloat16))
    assert_bf16(got, d["expected"], "golden transition (bf16 arithmetic)")


@pytest.mark.gpu
@pytest.mark.parametrize("autocast", [False, True])
def test_hip_reproduces_block_fixture(autocast):
    say(f"[gpu] golden block autocast={autocast}")
    mod, d, _ = loaded("block_n14_cz64_cs64")
    mod = mod.cuda()
    z0, s0 = d["z"].cuda(), d["s"].cuda()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        s, z = mod(s0, z0.clone(), d["mask"].cuda(), triangle_multiplicative="hip",
                   triangle_attention="hip", inplace_safe=True)
    if autocast:
        assert_bf16(z - z0, d["expected_z"] - d["z"], "golden block z update (bf16)")
        assert_bf16(s - s0, d["expected_s"] - d["s"], "golden block s update (bf16)")
    else:
        assert_fp32(z, d["expected_z"], "golden block z")
        assert_fp32(s, d["expected_s"], "golden block s")
