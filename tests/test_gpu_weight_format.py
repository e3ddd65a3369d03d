"""GPU parity of the weight-format tool: the inverse shuffles against the
oracle's restatements (bit for bit), the scale-buffer check on clean and
planted-defect buffers, and a weight written to a file, read back and fed to
the GEMM giving the same bytes as the operand it came from."""
import numpy as np
import pytest

import oracle
from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K", [(16, 64), (48, 192), (272, 512), (1040, 4096)])
def test_unshuffle_inverts_shuffle(dev, N, K):
    import torch

    import mbs_amd

    say(f"unshuffle N={N} K={K}")
    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s = rng.integers(0, 256, (N, K // 32), dtype=np.uint8)
    b_pre = oracle.shuffle_b(w)
    s_shuf = oracle.shuffle_scales(s, K, pad=127)
    got_w = mbs_amd.unshuffle_weight(torch.from_numpy(b_pre).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got_w, oracle.unshuffle_b(b_pre))
    np.testing.assert_array_equal(got_w, w)
    got_s = mbs_amd.unshuffle_scales(torch.from_numpy(s_shuf).to(dev), N, K).cpu().numpy()
    np.testing.assert_array_equal(got_s, oracle.unshuffle_scales(s_shuf, N, K))
    np.testing.assert_array_equal(got_s, s)
    # and the device shuffles invert the device unshuffles
    wt = torch.from_numpy(w).to(dev)
    np.testing.assert_array_equal(
        mbs_amd.unshuffle_weight(mbs_amd.shuffle_weight(wt)).cpu().numpy(), w)


@pytest.mark.parametrize("rows,K", [(1, 32), (33, 96), (256, 8192)])
def test_check_scales_counts_defects(dev, rows, K):
    import torch

    import mbs_amd

    say(f"check_scales rows={rows} K={K}")
    rng = np.random.default_rng(rows * 7 + K)
    s = rng.integers(0, 255, (rows, K // 32), dtype=np.uint8)  # no 0xFF
    buf = oracle.shuffle_scales(s, K, pad=127).reshape(-1).copy()
    t = torch.from_numpy(buf).to(dev)
    assert mbs_amd.check_scales(t, rows, K, 127) == (0, 0)
    # plant two NaN scale bytes among the live entries and, where the buffer
    # has padding, three wrong padding bytes
    snp = oracle.scale_pad(K)
    flat_s = oracle.lib().oracle_flat_s
    live = [flat_s(r, b, snp) for r, b in ((0, 0), (rows - 1, K // 32 - 1))]
    pad = [flat_s(r, b, snp) for r in range(oracle.round_up(rows, 32)) for b in range(snp)
           if r >= rows or b >= K // 32][:3]
    bad = buf.copy()
    bad[live] = 0xFF
    bad[pad] = 0x00
    t = torch.from_numpy(bad).to(dev)
    assert mbs_amd.check_scales(t, rows, K, 127) == (len(pad), len(set(live)))
    assert mbs_amd.check_scales(t, rows, K, -1) == (0, len(set(live)))


def test_weight_file_round_trip(dev, tmp_path):
    import torch

    import mbs_amd
    from mbs_amd import weight_format as wf

    say("weight file round trip")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    N, K, M = 256, 1024, 64
    w = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    for mbs in (False, True):
        op = wf.prepare_weight(w, mbs=mbs)
        wf.validate_weight(op["weight"], op["weight_scale"], N, K, op.get("weight_factor"))
        path = tmp_path / f"w{int(mbs)}.safetensors"
        wf.save_weight(path, op["weight"], op["weight_scale"], N, K, op.get("weight_factor"))
        back = wf.load_weight(path, device=dev)
        for k in ("weight", "weight_scale", "weight_factor"):
            if k in op:
                assert torch.equal(back[k], op[k]), k
        # unpack returns the plain quantizer output
        if mbs:
            packed, scale, _ = mbs_amd.quantize_mxfp4_mbs(w, shuffle=False)
        else:
            packed, scale = mbs_amd.quantize_mxfp4(w, shuffle=False)
        pw, ps = wf.unpack_weight(back["weight"], back["weight_scale"], N, K)
        assert torch.equal(pw, packed) and torch.equal(ps, scale)
        # the GEMM gives the same result from the file as from memory
        A, As = mbs_amd.quantize_mxfp4(x, shuffle=True)
        Af = torch.zeros(M, dtype=torch.uint8, device=dev) if mbs else None
        c0 = mbs_amd.gemm_a4w4(A, op["weight"], As, op["weight_scale"], Af, op.get("weight_factor"))
        c1 = mbs_amd.gemm_a4w4(A, back["weight"], As, back["weight_scale"], Af,
                               back.get("weight_factor"))
        assert torch.equal(c0, c1)


def test_validate_weight_reports_defects(dev):
    import torch

    from mbs_amd import weight_format as wf

    say("validate_weight defects")
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    N, K = 48, 256
    op = wf.prepare_weight((torch.randn(N, K, generator=g, device=dev)).to(torch.bfloat16))
    with pytest.raises(ValueError, match="shape"):
        wf.validate_weight(op["weight"][:32], op["weight_scale"], N, K)
    with pytest.raises(ValueError, match="bytes, need"):
        wf.validate_weight(op["weight"], op["weight_scale"].reshape(-1)[:100], N, K)
    s = op["weight_scale"].clone().reshape(-1)
    s[0] = 0xFF
    with pytest.raises(ValueError, match="0xFF"):
        wf.validate_weight(op["weight"], s, N, K)
    s = op["weight_scale"].clone()
    s[-1, -1] = 3  # a padding row (N=48 -> 64 rows)
    with pytest.raises(ValueError, match="padding"):
        wf.validate_weight(op["weight"], s, N, K)
    wf.validate_weight(op["weight"], s, N, K, pad_byte=None)
