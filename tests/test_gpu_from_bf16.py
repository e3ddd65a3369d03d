"""GPU parity of the decode GEMM from a bf16 activation (one launch: the
decode kernel quantizes x in registers) against the reference's two-step
flow, quantize then GEMM (test_gemm_a4w4.py:134-141, bench_one.py:19-30),
run with this library's quantizer and the same decode plan: the outputs must
be equal bit for bit, on every decode configuration, with and without K
splits, on the BASELINE decode shapes, K tails, special values (NaN, inf,
-0, subnormal, all-zero and saturated blocks) and the affine epilogue.  The
two-step path itself is checked against the CPU oracle elsewhere; here one
small case is also checked against the oracle directly."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu


def skinny_configs(M):
    import mbs_amd

    e = mbs_amd.ext()
    names = [e.config_name(c) for c in range(e.num_configs())]
    return [c for c, n in enumerate(names)
            if n.startswith("skinny") and M <= (16 if "_m16_" in n else 32)]


def operands(M, N, K, seed, dev):
    """bf16 x ~ N(0,1) with 1% outlier K-channels x20 (configs[2]'s rule),
    weights N(0, 0.02) quantized and preshuffled on the GPU."""
    import torch

    import mbs_amd

    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    cols = torch.randperm(K, generator=g)[: max(1, K // 100)]
    x[:, cols] *= 20
    w = torch.randn(N, K, generator=g) * 0.02
    x = x.to(torch.bfloat16).to(dev)
    wq, ws = mbs_amd.quantize_mxfp4(w.to(torch.bfloat16).to(dev))
    return x, mbs_amd.shuffle_weight(wq), ws


def two_step(x, B, Bs, config=-1, splits=0, alpha=1.0, bias=None):
    import mbs_amd

    A, As = mbs_amd.quantize_mxfp4(x)
    if config < 0:
        return mbs_amd.gemm_a4w4(A, B, As, Bs, alpha=alpha, bias=bias)
    return mbs_amd.ext().gemm_a4w4_config(config, splits, A, B, As, Bs, None, None, alpha, bias)


def same_bits(got, want, tag):
    import torch

    assert got.shape == want.shape, tag
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), tag


@pytest.mark.parametrize("M", [1, 4, 8, 16, 32])
def test_decode_shapes_default_plan(dev, M):
    """configs[2] shapes (and M = 8): one launch equals quantize + gemm_a4w4."""
    import mbs_amd

    N = K = 8192
    x, B, Bs = operands(M, N, K, 100 + M, dev)
    plan = mbs_amd.ext().plan_name(M, N, K)
    assert plan.startswith("skinny"), plan
    say(f"from_bf16 default plan M={M} N={N} K={K} ({plan})")
    got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, one_launch=True)
    same_bits(got, two_step(x, B, Bs), f"M={M}")
    again = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, one_launch=True)
    same_bits(again, got, f"M={M} repeat")
    # the default form (one launch up to M = 4, two above) gives the same bytes
    same_bits(mbs_amd.gemm_a4w4_from_bf16(x, B, Bs), got, f"M={M} default")


@pytest.mark.parametrize("M,N,K", [(1, 256, 512), (3, 1280, 576), (2, 4096, 4160),
                                   (8, 1280, 576), (6, 96, 64),
                                   (17, 2112, 7168), (32, 1280, 576),
                                   (5, 4096, 4160), (32, 48, 64)])
def test_every_decode_config_and_split(dev, M, N, K):
    """Forced decode configurations and split counts (K tails included: 576
    and 4160 end in a half stage; 64 is one half stage)."""
    import mbs_amd

    x, B, Bs = operands(M, N, K, M * 7 + N + K, dev)
    for c in skinny_configs(M):
        for splits in (0, 1, 2, 3):
            say(f"from_bf16 config={mbs_amd.ext().config_name(c)} splits={splits} M={M} N={N} K={K}")
            got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, config=c, splits=splits)
            same_bits(got, two_step(x, B, Bs, c, splits), f"config {c} splits {splits}")


def test_special_values(dev):
    """NaN, +-inf, -0, negative values that round to zero, subnormals, all-zero
    and saturating blocks in the activation; bit patterns compared (NaN
    outputs included)."""
    import torch

    import mbs_amd

    M, N, K = 8, 512, 1024
    rng = np.random.default_rng(7)
    bits = (rng.standard_normal((M, K)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    bits[0, 3] = 0x7FC1                     # NaN: block scale 255, codes 0
    bits[1, 40] = 0xFF80                    # -inf
    bits[1, 100] = 0x7F80                   # +inf
    bits[2, :64] = 0x8000                   # -0 blocks
    bits[3, :32] = 0x8001                   # negative subnormals
    bits[3, 32:64] = 0                      # all-zero block
    bits[4, :32] = 0x7F7F                   # largest finite: saturating block
    bits[5, :16] = 0x0001                   # tiny values beside a huge one
    bits[5, 16] = 0x7F00
    bits[6, 200:232] = 0xB000               # small negatives (-2^-31)
    x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev)
    _, B, Bs = operands(1, N, K, 11, dev)
    for c in skinny_configs(M):
        say(f"from_bf16 specials config={mbs_amd.ext().config_name(c)}")
        got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, config=c)
        same_bits(got, two_step(x, B, Bs, c), f"config {c}")
    out = bf16_to_f32(got)
    assert np.isfinite(out[[2, 3, 7]]).all()   # -0, subnormal / all-zero, plain rows


def test_affine_epilogue(dev):
    """alpha and a bias row: equal to quantize + the affine gemm_a4w4."""
    import torch

    import mbs_amd

    M, N, K = 16, 2048, 4096
    x, B, Bs = operands(M, N, K, 21, dev)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(3)) * 4).to(torch.bfloat16).to(dev)
    for alpha, b in [(0.5, None), (1.0, bias), (-3.25, bias)]:
        say(f"from_bf16 affine alpha={alpha} bias={b is not None}")
        got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, alpha=alpha, bias=b, one_launch=True)
        same_bits(got, two_step(x, B, Bs, alpha=alpha, bias=b), f"alpha {alpha}")


def test_oracle_small(dev):
    """One small case straight against the CPU oracle (quantize, dequantize,
    fp32 matmul, bf16) at the north-star tolerance; the two-step path's
    quantized bytes (which the one-launch output equals through) match the
    oracle's bit for bit."""
    import mbs_amd

    M, N, K = 3, 96, 1088
    x, B, Bs = operands(M, N, K, 5, dev)
    say(f"from_bf16 oracle M={M} N={N} K={K}")
    got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, one_launch=True)
    xf = x.float().cpu().numpy()
    xq, xs = oracle.quantize_mxfp4(xf)
    wq = oracle.unshuffle_b(B.cpu().numpy())
    ws = oracle.unshuffle_scales(Bs.cpu().numpy(), N, K)
    ref = oracle.epilogue_bf16(oracle.gemm_f32_small(oracle.dequant_mxfp4(xq, xs),
                                                     oracle.dequant_mxfp4(wq, ws)))
    g = bf16_to_f32(got)
    assert_close(g, oracle.bf16_bits_to_f32(ref), "from_bf16 vs oracle")
    A, As = mbs_amd.quantize_mxfp4(x)
    np.testing.assert_array_equal(A.cpu().numpy(), xq)
    np.testing.assert_array_equal(oracle.unshuffle_scales(As.cpu().numpy(), M, K), xs)
    same_bits(got, two_step(x, B, Bs), "from_bf16 vs two-step")


def test_large_m_and_empty(dev):
    """M > 32 runs the two launches (same bytes) and refuses the one-launch
    form; M == 0 returns an empty result without launching."""
    import torch

    import mbs_amd

    x, B, Bs = operands(64, 256, 512, 9, dev)
    say("from_bf16 M=64 (two launches)")
    same_bits(mbs_amd.gemm_a4w4_from_bf16(x, B, Bs), two_step(x, B, Bs), "M=64")
    with pytest.raises(RuntimeError, match="M <= 32"):
        mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, one_launch=True)
    empty = torch.empty(0, 512, dtype=torch.bfloat16, device=dev)
    say("from_bf16 M=0")
    assert mbs_amd.gemm_a4w4_from_bf16(empty, B, Bs, one_launch=True).shape == (0, 256)


def sixteen_row_configs():
    import mbs_amd

    e = mbs_amd.ext()
    return [c for c in range(e.num_configs()) if e.config_name(c).startswith("skinny_m16_")]


def two_step_mbs(x, B, Bs, Bf, config=-1, alpha=1.0, bias=None):
    """The reference's MBS decode flow: MBS-quantize the activation (factor
    byte per row), then the factor GEMM with both factors."""
    import mbs_amd

    A, As, Af = mbs_amd.quantize_mxfp4_mbs(x)
    if config < 0:
        return mbs_amd.gemm_a4w4(A, B, As, Bs, Af, Bf, alpha=alpha, bias=bias)
    return mbs_amd.ext().gemm_a4w4_config(config, 1, A, B, As, Bs, Af, Bf, alpha, bias)


@pytest.mark.parametrize("M,N,K", [(1, 8192, 8192), (4, 8192, 8192), (8, 8192, 8192),
                                   (3, 1280, 576), (6, 96, 64), (5, 4096, 4160)])
def test_mbs_activation_one_launch(dev, M, N, K):
    """With the weights' MBS factors the one-launch form MBS-quantizes the
    activation (each workgroup derives the row factor bytes from the rows'
    maxima over all of K) and applies both factors: equal, bit for bit, to
    quantize_mxfp4_mbs followed by the factor GEMM on the same plan."""
    import torch

    import mbs_amd

    x, B, Bs = operands(M, N, K, 300 + M * 3 + K, dev)
    Bf = torch.randint(0, 256, (N,), dtype=torch.uint8,
                       generator=torch.Generator().manual_seed(M + N)).to(dev)
    for c in sixteen_row_configs():
        say(f"from_bf16 MBS config={mbs_amd.ext().config_name(c)} M={M} N={N} K={K}")
        got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, config=c, B_factor=Bf)
        same_bits(got, two_step_mbs(x, B, Bs, Bf, c), f"MBS config {c}")
    if "splits=1" in mbs_amd.ext().plan_name(M, N, K):
        say(f"from_bf16 MBS default plan M={M}")
        got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, B_factor=Bf, one_launch=True)
        same_bits(got, two_step_mbs(x, B, Bs, Bf), "MBS default plan")
        same_bits(mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, B_factor=Bf), got, "MBS default form")


def test_mbs_activation_specials_and_affine(dev):
    """Rows whose maximum is zero, infinite or NaN (factor byte 0), a row of
    tiny values (a large factor) and the affine epilogue with MBS factors."""
    import torch

    import mbs_amd

    M, N, K = 8, 512, 1024
    rng = np.random.default_rng(17)
    bits = (rng.standard_normal((M, K)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    bits[0, :] = 0                         # all-zero row
    bits[1, 77] = 0x7F80                   # +inf in the row
    bits[2, 5] = 0xFFC0                    # NaN in the row
    bits[3, :] = (bits[3, :] & 0x8000) | 0x2000   # tiny values: max far below 6
    bits[4, 0] = 0x7F7F                    # the largest finite value
    x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev)
    _, B, Bs = operands(1, N, K, 23, dev)
    Bf = torch.randint(0, 256, (N,), dtype=torch.uint8, generator=torch.Generator().manual_seed(5)).to(dev)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(6)) * 3).to(torch.bfloat16).to(dev)
    for c in sixteen_row_configs():
        for alpha, b in [(1.0, None), (0.75, bias)]:
            say(f"from_bf16 MBS specials config={mbs_amd.ext().config_name(c)} alpha={alpha}")
            got = mbs_amd.gemm_a4w4_from_bf16(x, B, Bs, alpha=alpha, bias=b, config=c, B_factor=Bf)
            same_bits(got, two_step_mbs(x, B, Bs, Bf, c, alpha, b), f"MBS specials config {c}")
    with pytest.raises(RuntimeError, match="M <= 8"):
        xs, _, _ = operands(9, N, K, 1, dev)
        mbs_amd.gemm_a4w4_from_bf16(xs, B, Bs, B_factor=Bf, one_launch=True)
