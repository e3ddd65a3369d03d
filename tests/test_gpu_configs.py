"""The five BASELINE configurations at their full sizes, through the C ABI.

Inputs come from the seeded generators (mbs_amd.synthetic) quantized by the
CPU oracle.  Where the CPU oracle finishes in seconds it checks every element
(config 0, 2, and 3 at M=256); for the larger problems it checks a sample of
rows (first, last, tails, random) and the whole output is compared with the
reference's own dequantize-then-fp32-matmul path run on the GPU (our
dequantizer, bit-checked against the oracle on the sampled rows, followed by
torch.mm in fp32).  Size-independent properties close the rest: repeat runs
are bit-identical, and raising every A scale byte by one doubles the output
exactly."""
import numpy as np
import pytest

import oracle
from gpu_util import Case, assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu

FULL_ORACLE_FLOP = 8e9   # full CPU check below this many flops


def make_case(cfg, M, N, K, factors=False):
    from mbs_amd import synthetic

    x, w = synthetic.make_operands(cfg, M, N, K)
    f = None
    if factors:
        af, bf = synthetic.make_factors(M, N, 3000 + cfg)
        f = (af.numpy().reshape(-1), bf.numpy().reshape(-1))
    return Case.from_bf16(x, w, factors=f)


def sample_rows(M, n=48, seed=0):
    rng = np.random.default_rng(seed)
    fixed = {0, 1, 15, 16, 31, 32, M // 2, M - 33, M - 17, M - 16, M - 2, M - 1}
    rows = sorted({r for r in fixed if 0 <= r < M} | set(rng.integers(0, M, n).tolist()))
    return np.array(rows)


def gpu_reference(c):
    """Dequantize on the GPU, fp32 torch.mm on the GPU, epilogue on the host."""
    import torch

    import mbs_amd

    a = mbs_amd.dequant_mxfp4(c.A, c.As, False)
    b = mbs_amd.dequant_mxfp4(c.B, c.Bs, True)
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        cf = torch.mm(a, b.T).cpu().numpy()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    return a, oracle.bf16_bits_to_f32(oracle.epilogue_bf16(cf, c.a_factor, c.b_factor))


def check_case(c, tag):
    M, N, K = c.M, c.N, c.K
    say(f"{tag}: kernel run M={M} N={N} K={K}")
    out = c.run()
    got = bf16_to_f32(out)[:M]
    if 2.0 * M * N * K <= FULL_ORACLE_FLOP:
        say(f"{tag}: full CPU oracle")
        assert_close(got, oracle.bf16_bits_to_f32(c.reference()), f"{tag} full")
    else:
        rows = sample_rows(M)
        say(f"{tag}: CPU oracle on {len(rows)} rows")
        assert_close(got[rows], oracle.bf16_bits_to_f32(c.reference(rows)), f"{tag} rows")
        say(f"{tag}: GPU dequant + fp32 mm reference")
        a_deq, ref = gpu_reference(c)
        a_rows = a_deq[torch_index(rows)].cpu().numpy()
        np.testing.assert_array_equal(
            a_rows.view(np.uint32),
            oracle.dequant_mxfp4(c.x_packed[rows], c.x_scales[rows]).view(np.uint32))
        assert_close(got, ref, f"{tag} gpu-ref")
    say(f"{tag}: determinism")
    again = bf16_to_f32(c.run())[:M]
    np.testing.assert_array_equal(got, again)
    return got


def torch_index(rows):
    import torch

    return torch.from_numpy(rows).cuda()


def test_cfg0(dev):
    from mbs_amd import synthetic

    (M, N, K), = synthetic.config_shapes(0)
    check_case(make_case(0, M, N, K), "cfg0")
    check_case(make_case(0, M, N, K, factors=True), "cfg0+factors")


def test_cfg1_8192_cubed(dev):
    c = make_case(1, 8192, 8192, 8192)
    got = check_case(c, "cfg1")
    # raising every A scale byte by one doubles the output exactly
    import torch

    say("cfg1: scale-doubling property")
    c.As = (c.As.to(torch.int16) + 1).clamp(max=254).to(torch.uint8)
    doubled = bf16_to_f32(c.run())[: c.M]
    fin = np.isfinite(got) & (np.abs(got) < 1e38)
    np.testing.assert_array_equal(doubled[fin], 2 * got[fin])


@pytest.mark.parametrize("M", [1, 4, 16, 32])
def test_cfg2_decode(dev, M):
    check_case(make_case(2, M, 8192, 8192, factors=(M == 16)), f"cfg2 M={M}")


@pytest.mark.parametrize("M", [256, 2048])
@pytest.mark.parametrize("NK", [(7168, 2048), (4096, 7168), (2112, 7168)])
def test_cfg3_moe_shapes(dev, M, NK):
    N, K = NK
    check_case(make_case(3, M, N, K, factors=(N == 4096)), f"cfg3 M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [1000, 3333])
@pytest.mark.parametrize("N", [1280, 5120])
@pytest.mark.parametrize("K", [512, 12288])
def test_cfg4_ragged(dev, M, N, K):
    c = make_case(4, M, N, K, factors=(M == 1000 and N == 1280))
    # the generator injects all-zero and saturated blocks on both operands
    assert (c.x_scales == 0).any() and (c.w_scales == 0).any()
    check_case(c, f"cfg4 M={M} N={N} K={K}")
