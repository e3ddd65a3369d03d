"""Write the committed golden vectors (run from the repo root):

    python tests/golden/make_golden.py

* ``cfg0.npz`` -- configuration 0 (M=128, N=256, K=512) end to end: the
  seeded bf16 operands (as bit patterns), their MXFP4 bytes (packed, plain
  scales, shuffled scales, preshuffled B), MBS factor bytes, and the bf16
  results of the reference oracle without and with factors
  (test_gemm_a4w4.py:28-44, 54-69 of the reference, restated by ``oracle``).
* ``synthetic_sha256.json`` -- SHA-256 of the quantized bytes of every shape
  of configurations 1-4, to detect drift of the seeded generators.

The vectors come from this repository's oracle, whose functions are pinned
independently (tests/test_oracle_*.py); the reference ships no golden data
of its own for this path.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from mbs_amd import synthetic  # noqa: E402

FACTOR_SEED = 2000


def bf16_bits(t):
    import torch

    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def quantize(t):
    return oracle.quantize_mxfp4(t.float().numpy())


def make_cfg0():
    M, N, K = synthetic.CFG0["M"], synthetic.CFG0["N"], synthetic.CFG0["K"]
    x, w = synthetic.make_operands(0, M, N, K)
    xp, xs = quantize(x)
    wp, ws = quantize(w)
    af, bf = synthetic.make_factors(M, N, FACTOR_SEED)
    af, bf = af.numpy().reshape(-1), bf.numpy().reshape(-1)
    return dict(
        M=np.int64(M), N=np.int64(N), K=np.int64(K),
        x_bits=bf16_bits(x), w_bits=bf16_bits(w),
        x_packed=xp, x_scales=xs, w_packed=wp, w_scales=ws,
        w_shuffled=oracle.shuffle_b(wp),
        x_scales_shuffled=oracle.shuffle_scales(xs, K),
        w_scales_shuffled=oracle.shuffle_scales(ws, K),
        a_factor=af, b_factor=bf,
        c_bf16=oracle.run_torch(xp, wp, xs, ws),
        c_mbs_bf16=oracle.run_torch(xp, wp, xs, ws, af, bf),
    )


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def synthetic_hashes():
    out = {}
    for cfg in (1, 2, 3, 4):
        for (M, N, K) in synthetic.config_shapes(cfg):
            x, w = synthetic.make_operands(cfg, M, N, K)
            xp, xs = quantize(x)
            wp, ws = quantize(w)
            out[f"cfg{cfg}_{M}x{N}x{K}"] = dict(x_packed=sha(xp), x_scales=sha(xs),
                                                w_packed=sha(wp), w_scales=sha(ws))
    return out


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "cfg0.npz"), **make_cfg0())
    with open(os.path.join(HERE, "synthetic_sha256.json"), "w") as f:
        json.dump(synthetic_hashes(), f, indent=1, sort_keys=True)
    print("wrote cfg0.npz and synthetic_sha256.json")
