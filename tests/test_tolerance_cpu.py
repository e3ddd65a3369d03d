"""The north-star tolerance (|err| <= 1e-2 * max|C_ref| + 1 bf16 ulp, written
in gpu_util.assert_close) is strict enough to catch a plausible kernel bug
and loose enough for legitimate rounding differences, at configs[1]'s N and K
(8192 x 8192, the seeded configs[1] operands with their outlier channels),
on 64 rows of A so the CPU oracle finishes in seconds:

* an output whose contraction skipped one 32-wide K block (a dropped MFMA
  K-step, the mistake a wrong stage count or K-tail mask would make) fails,
  for ordinary blocks and for a block holding an outlier channel;
* an output that differs from the oracle by one bf16 ulp everywhere passes.

The bad outputs are planted in the oracle's inputs (CPU only)."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_close

ROWS = 64


@pytest.fixture(scope="module")
def cfg1_rows():
    from mbs_amd import synthetic

    x, w = synthetic.make_operands(1, 8192, 8192, 8192)
    xp, xs = oracle.quantize_mxfp4(x[:ROWS].float().numpy())
    wp, ws = oracle.quantize_mxfp4(w.float().numpy())
    ref = oracle.bf16_bits_to_f32(oracle.run_torch(xp, wp, xs, ws))
    # K-blocks of A's first rows that hold an outlier channel (x20 columns)
    big = np.abs(x[:ROWS].float().numpy()).max(axis=0) > 8.0
    outlier_blocks = np.unique(np.nonzero(big)[0] // 32)
    return xp, xs, wp, ws, ref, outlier_blocks


def _drop_block(xp, kb):
    bad = xp.copy()
    bad[:, kb * 16:(kb + 1) * 16] = 0     # e2m1 code 0 in both nibbles: 16 bytes = 32 values
    return bad


@pytest.mark.parametrize("kind", ["ordinary", "outlier"])
def test_dropped_k_block_is_rejected(cfg1_rows, kind):
    xp, xs, wp, ws, ref, outlier_blocks = cfg1_rows
    assert len(outlier_blocks) > 0
    blocks = [0, 97, 255] if kind == "ordinary" else list(outlier_blocks[:2])
    for kb in blocks:
        got = oracle.bf16_bits_to_f32(oracle.run_torch(_drop_block(xp, int(kb)), wp, xs, ws))
        with pytest.raises(AssertionError, match="out of tolerance"):
            assert_close(got, ref, f"block {kb} dropped")


def test_one_ulp_everywhere_is_accepted(cfg1_rows):
    *_, ref, _ = cfg1_rows
    bits = oracle.f32_to_bf16_bits(ref)
    nz = bits & 0x7FFF != 0
    up = np.where(nz, bits + 1, bits).astype(np.uint16)      # one ulp away from zero
    assert_close(oracle.bf16_bits_to_f32(up), ref, "one ulp")
