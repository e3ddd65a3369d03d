"""GPU parity of the grouped (mixture-of-experts) GEMM: one launch over E
experts against E separate dense launches on the same bytes (bit for bit:
the per-element accumulation order does not depend on the tile), and against
the oracle's run_torch per expert.  Covers every
grouped configuration, empty experts, many small experts, MBS factors, a
64-wide K tail, offsets given on the device, alpha with a bias per expert,
and the host-side checks."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu


def make_problem(rng, rows, N, K, factors=False):
    """Expert row counts `rows` (multiples of 32) -> host bytes of A (all
    experts' rows stacked), the E weight matrices and their scales."""
    M = int(sum(rows))
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((len(rows), N, K)) * 0.05).astype(np.float32)
    xp, xs = oracle.quantize_mxfp4(x)
    wq = [oracle.quantize_mxfp4(w[e]) for e in range(len(rows))]
    af = rng.integers(0, 256, M, dtype=np.uint8) if factors else None
    bf = rng.integers(0, 256, (len(rows), N), dtype=np.uint8) if factors else None
    offs = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    return M, xp, xs, wq, af, bf, offs


def device_operands(dev, M, N, K, xp, xs, wq, af, bf):
    import torch

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    A = t(xp)
    As = t(oracle.shuffle_scales(xs, K, pad=127))
    B = t(np.stack([oracle.shuffle_b(wp) for wp, _ in wq]))
    Bs = t(np.stack([oracle.shuffle_scales(ws, K, pad=127).reshape(-1) for _, ws in wq]))
    Af = None if af is None else t(af)
    Bf = None if bf is None else t(bf.reshape(-1))
    return A, As, B, Bs, Af, Bf


def dense_expert(dev, e, offs, N, K, xp, xs, wq, af, bf):
    """The dense launch of expert e alone (its rows of A, its weights)."""
    import torch

    import mbs_amd

    r0, r1 = offs[e], offs[e + 1]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    A = t(xp[r0:r1])
    As = t(oracle.shuffle_scales(xs[r0:r1], K, pad=127))
    B = t(oracle.shuffle_b(wq[e][0]))
    Bs = t(oracle.shuffle_scales(wq[e][1], K, pad=127))
    Af = None if af is None else t(af[r0:r1])
    Bf = None if bf is None else t(bf[e])
    return mbs_amd.gemm_a4w4(A, B, As, Bs, Af, Bf)


@pytest.mark.parametrize("config", [0, 1, 2, 3])
@pytest.mark.parametrize("rows,N,K", [([64, 0, 96, 32], 512, 1024), ([256, 128], 256, 2048)])
def test_grouped_matches_dense_per_expert(dev, config, rows, N, K):
    import torch

    import mbs_amd

    name = mbs_amd.ext().grouped_config_name(config)
    say(f"grouped config={name} rows={rows} N={N} K={K}")
    rng = np.random.default_rng(len(rows) * 100 + N + K + config)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, rows, N, K)
    A, As, B, Bs, Af, Bf = device_operands(dev, M, N, K, xp, xs, wq, af, bf)
    got = mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.from_numpy(offs), config=config)
    torch.cuda.synchronize()
    for e in range(len(rows)):
        if rows[e] == 0:
            continue
        want = dense_expert(dev, e, offs, N, K, xp, xs, wq, af, bf)
        assert torch.equal(got[offs[e]:offs[e + 1]], want), (name, e)
        ref = oracle.bf16_bits_to_f32(oracle.run_torch(xp[offs[e]:offs[e + 1]], wq[e][0],
                                                       xs[offs[e]:offs[e + 1]], wq[e][1]))
        assert_close(bf16_to_f32(got[offs[e]:offs[e + 1]]), ref, f"{name} expert {e}")


@pytest.mark.parametrize("rows,N,K,factors", [
    ([32] * 24, 256, 512, False),              # many small experts (one partial tile each)
    ([96, 160, 0, 32, 224], 768, 1088, True),  # factors, K % 128 == 64 (K tail)
    ([0, 0, 288], 1024, 4096, True),           # leading empty experts
    ([256] * 8, 7168, 2048, False),            # configs[3] expert shapes: the tuned-table
    ([256] * 8, 2112, 7168, False),            # plans (256x256 and 128x256)
])
def test_grouped_default_plan(dev, rows, N, K, factors):
    import torch

    import mbs_amd

    say(f"grouped default rows={rows[:6]}.. E={len(rows)} N={N} K={K} factors={factors}")
    rng = np.random.default_rng(sum(rows) + N + K)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, rows, N, K, factors)
    A, As, B, Bs, Af, Bf = device_operands(dev, M, N, K, xp, xs, wq, af, bf)
    goff = torch.from_numpy(offs).to(dev)       # offsets already on the device
    got = mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, goff, Af, Bf)
    torch.cuda.synchronize()
    for e in range(len(rows)):
        if rows[e] == 0:
            continue
        r0, r1 = offs[e], offs[e + 1]
        want = dense_expert(dev, e, offs, N, K, xp, xs, wq, af, bf)
        assert torch.equal(got[r0:r1], want), e
        ref = oracle.bf16_bits_to_f32(oracle.run_torch(
            xp[r0:r1], wq[e][0], xs[r0:r1], wq[e][1],
            None if af is None else af[r0:r1], None if bf is None else bf[e]))
        assert_close(bf16_to_f32(got[r0:r1]), ref, f"expert {e}")


@pytest.mark.parametrize("config", [0, 1, 2, 3])
def test_grouped_alpha_bias(dev, config):
    """Affine epilogue per expert: bf16(C * alpha * f(a) * f(b) + bias[e]) --
    the dense launch of each expert with its own bias row, bit for bit, and
    the oracle's epilogue within tolerance."""
    import torch

    import mbs_amd

    rows, N, K = [64, 0, 96, 32], 512, 1024
    name = mbs_amd.ext().grouped_config_name(config)
    say(f"grouped alpha/bias config={name} rows={rows} N={N} K={K}")
    rng = np.random.default_rng(77 + config)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, rows, N, K, factors=True)
    A, As, B, Bs, Af, Bf = device_operands(dev, M, N, K, xp, xs, wq, af, bf)
    bias = oracle.f32_to_bf16_bits((rng.standard_normal((len(rows), N)) * 2).astype(np.float32))
    bias_t = torch.from_numpy(bias.view(np.int16)).to(dev).view(torch.bfloat16)
    got = mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.from_numpy(offs), Af, Bf, config=config,
                                    alpha=-0.75, bias=bias_t)
    torch.cuda.synchronize()
    for e in range(len(rows)):
        if rows[e] == 0:
            continue
        r0, r1 = offs[e], offs[e + 1]
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        want = mbs_amd.gemm_a4w4(t(xp[r0:r1]), t(oracle.shuffle_b(wq[e][0])),
                                 t(oracle.shuffle_scales(xs[r0:r1], K, pad=127)),
                                 t(oracle.shuffle_scales(wq[e][1], K, pad=127)), t(af[r0:r1]), t(bf[e]),
                                 alpha=-0.75, bias=bias_t[e])
        assert torch.equal(got[r0:r1], want), (name, e)
        c32 = (oracle.dequant_mxfp4(xp[r0:r1], xs[r0:r1]).astype(np.float64)
               @ oracle.dequant_mxfp4(wq[e][0], wq[e][1]).astype(np.float64).T).astype(np.float32)
        ref = oracle.bf16_bits_to_f32(oracle.epilogue_affine_bf16(c32, af[r0:r1], bf[e], -0.75, bias[e]))
        assert_close(bf16_to_f32(got[r0:r1]), ref, f"{name} expert {e}")
    with pytest.raises(RuntimeError, match="bias"):
        mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.from_numpy(offs), bias=bias_t[0])


def test_grouped_rejects_bad_offsets(dev):
    import torch

    import mbs_amd

    say("grouped offset checks")
    rng = np.random.default_rng(1)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, [64, 64], 256, 512)
    A, As, B, Bs, _, _ = device_operands(dev, M, 256, 512, xp, xs, wq, None, None)
    for bad in ([0, 48, 128], [0, 96, 64], [32, 64, 128], [0, 64, 160]):
        with pytest.raises(RuntimeError, match="group_offsets"):
            mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.tensor(bad, dtype=torch.int32))
