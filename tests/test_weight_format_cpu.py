"""Host-side parts of the weight-format tool: the file container (metadata,
byte-exact tensors, format tag) and the structural checks that need no GPU."""
import numpy as np
import pytest
import torch

from mbs_amd import weight_format as wf


def test_file_container_round_trip(tmp_path):
    rng = np.random.default_rng(3)
    N, K = 48, 256
    w = torch.from_numpy(rng.integers(0, 256, (N, K // 2), dtype=np.uint8))
    s = torch.from_numpy(rng.integers(0, 256, (64, 8), dtype=np.uint8))
    f = torch.from_numpy(rng.integers(0, 256, (N,), dtype=np.uint8))
    p = tmp_path / "w.safetensors"
    wf.save_weight(p, w, s, N, K, f, pad_byte=127, validate=False)
    back = wf.read_weight_file(p)
    assert (back["N"], back["K"], back["scale_pad_byte"]) == (N, K, 127)
    assert torch.equal(back["weight"], w) and torch.equal(back["weight_scale"], s)
    assert torch.equal(back["weight_factor"], f)


def test_foreign_file_is_refused(tmp_path):
    from safetensors.torch import save_file

    p = tmp_path / "x.safetensors"
    save_file({"weight": torch.zeros(16, 32, dtype=torch.uint8)}, str(p), metadata={"format": "other"})
    with pytest.raises(ValueError, match="format"):
        wf.read_weight_file(p)


def test_validate_needs_device_tensors():
    w = torch.zeros(16, 32, dtype=torch.uint8)
    s = torch.zeros(32, 8, dtype=torch.uint8)
    with pytest.raises(ValueError, match="not on a GPU"):
        wf.validate_weight(w, s, 16, 64)
    with pytest.raises(ValueError, match="1-byte"):
        wf.validate_weight(w.float(), s, 16, 64)
