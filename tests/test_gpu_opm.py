"""GPU parity of the OuterProductMean kernels (the MSA module's MSA -> pair
update, triangular/layers.py:497-627; MSABlock builds it with c_m = 64,
c_hidden = 32 and c_z = 128, pairformer.py:799-803).

The HIP path computes in bf16 (the reference's bf16 mode); it is compared
with the CPU oracle in fp32 on the same bf16-rounded MSA at the bf16 tier
(rel-L2 <= 1e-2, max-abs <= 5e-2 after scaling the update to O(1)), at
shapes covering the padding of residues (to 64) and MSA rows (to 64), the
workgroup-to-XCD tile map, every c_m and c_z, masked MSA rows and residues,
no MSA rows, and the fused residual add.  At the MSA module's size the
oracle is the module's own torch path in fp32 on the GPU.
"""

import pytest
import torch

from helpers import assert_bf16, params_of, say, seeded
from oracle import reference as ref
from opendde_amd import _lib
from opendde_amd.outer_product_mean import OuterProductMean

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _fp32_matmul():
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = old
    torch.cuda.synchronize()


def _module(c_m, c_z, seed):
    # weights ~ N(0, 0.1^2) and a non-zero output bias: the update is O(1)
    # after the division by the mask counts
    mod = seeded(OuterProductMean(c_m, c_z, 32), seed, 0.1)
    with torch.no_grad():
        mod.linear_out.bias.normal_(0.0, 0.1, generator=torch.Generator().manual_seed(seed))
    return mod


def _inputs(S, N, c_m, seed, masked):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(S, N, c_m, generator=g).to(torch.bfloat16)
    mask = None
    if masked:
        mask = (torch.rand(S, N, generator=g) > 0.2).float()
    return m, mask


CASES = [
    # S, N, c_m, c_z, masked
    (5, 17, 64, 128, True),
    (37, 40, 32, 64, False),
    (130, 72, 128, 384, True),
    (64, 130, 64, 256, True),
    (70, 100, 64, 128, True),   # residues padded to 128: the 8 x 8 band tile map
    (200, 64, 64, 128, False),
]


@pytest.mark.parametrize("S,N,c_m,c_z,masked", CASES)
def test_outer_product_mean_matches_oracle(S, N, c_m, c_z, masked):
    say(f"[gpu] opm S={S} N={N} c_m={c_m} c_z={c_z} mask={masked}")
    mod = _module(c_m, c_z, 900 + S + N + c_z)
    m, mask = _inputs(S, N, c_m, 40 + S, masked)
    exp = ref.outer_product_mean(m.float(), mask, params_of(mod))
    mod = mod.to(DEV)
    before = _lib.launch_count(_lib.K_OPM)
    got = mod(m.to(DEV), None if mask is None else mask.to(DEV), kernel="hip")
    torch.cuda.synchronize()
    assert _lib.launch_count(_lib.K_OPM) == before + 1
    assert got.dtype == torch.bfloat16 and got.shape == (N, N, c_z)
    assert_bf16(got.float(), exp, f"opm S={S} N={N} c_m={c_m} c_z={c_z}")


def test_outer_product_mean_fp32_msa_under_autocast_and_residual_add():
    """fp32 MSA under bf16 autocast, and the MSA module's z += update fused
    into the kernel for an fp32 and a bf16 pair tensor."""
    S, N, c_m, c_z = 48, 33, 64, 128
    say("[gpu] opm autocast + residual")
    mod = _module(c_m, c_z, 950)
    g = torch.Generator().manual_seed(951)
    m = torch.randn(S, N, c_m, generator=g)
    mask = (torch.rand(S, N, generator=g) > 0.3).float()
    z = torch.randn(N, N, c_z, generator=g)
    exp = ref.outer_product_mean(m, mask, params_of(mod))
    mod = mod.to(DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        got = mod(m.to(DEV), mask.to(DEV), kernel="hip")
        assert_bf16(got.float(), exp, "opm under autocast")
        for zdt in (torch.float32, torch.bfloat16):
            zg = z.to(DEV, zdt)
            z0 = zg.float().clone()
            out = mod.hip_apply(m.to(DEV), mask.to(DEV), out=zg, add_residual=True)
            assert out.data_ptr() == zg.data_ptr()
            assert_bf16(zg.float() - z0, exp, f"opm residual add into {zdt}")


def test_outer_product_mean_masked_rows_columns_and_no_msa():
    """A fully masked residue gets norm eps (update = b_out / eps there, as
    in the reference); a fully masked MSA row contributes nothing; with no
    MSA rows at all the update is b_out / eps everywhere."""
    S, N, c_m, c_z = 20, 24, 64, 64
    say("[gpu] opm masked residues / rows, empty MSA")
    mod = _module(c_m, c_z, 960)
    m, mask = _inputs(S, N, c_m, 961, True)
    mask[:, 5] = 0.0
    mask[7, :] = 0.0
    p = params_of(mod)
    exp = ref.outer_product_mean(m.float(), mask, p)
    dmod = mod.to(DEV)
    got = dmod(m.to(DEV), mask.to(DEV), kernel="hip").float().cpu()
    # scale: the rows of residue 5 hold b_out / eps (~100); compare each part
    # at its own magnitude
    keep = torch.ones(N, dtype=torch.bool)
    keep[5] = False
    assert_bf16(got[keep][:, keep], exp[keep][:, keep], "opm unmasked pairs")
    torch.testing.assert_close(got[5], exp[5], rtol=1e-2, atol=1e-2)
    empty = dmod(m[:0].to(DEV), mask[:0].to(DEV), kernel="hip").float().cpu()
    torch.testing.assert_close(empty, (p["linear_out.bias"] / ref.OPM_EPS).expand(N, N, c_z),
                               rtol=1e-2, atol=1e-2)


def test_outer_product_mean_msa_module_size_vs_gpu_fp32():
    """S = 512 MSA rows, N = 384 residues, c_m = 64, c_z = 128 (the MSA
    module's widths) against the module's torch path in fp32 on the GPU; and
    repeated calls are bitwise identical."""
    S, N, c_m, c_z = 512, 384, 64, 128
    say(f"[gpu] opm S={S} N={N}")
    mod = _module(c_m, c_z, 970).to(DEV)
    g = torch.Generator().manual_seed(971)
    m = torch.randn(S, N, c_m, generator=g).to(torch.bfloat16).to(DEV)
    mask = (torch.rand(S, N, generator=g) > 0.1).float().to(DEV)
    with torch.no_grad():
        exp = mod(m.float(), mask, chunk_size=64)
        got = mod(m, mask, kernel="hip")
        again = mod(m, mask, kernel="hip")
    torch.cuda.synchronize()
    assert_bf16(got.float(), exp, "opm msa-module size")
    assert torch.equal(got, again)


def test_outer_product_mean_rejects_fp32_compute():
    mod = _module(64, 128, 980).to(DEV)
    m = torch.randn(8, 8, 64, device=DEV)
    with pytest.raises(NotImplementedError):
        mod(m, kernel="hip")
