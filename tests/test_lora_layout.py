"""Host-side layout of LoRA B for the fused consumers (no GPU needed)."""

import pytest
import torch

from pagelora_amd.fused_ops import lora_b_chunk8


def test_lora_b_chunk8_layout():
    # element (a, j, i, k, l, e) of the chunked layout is B[a][8(64j + l) + i][8k + e],
    # zero past out_features (here 600 columns: one full 512-column block and a padded one)
    out, r = 600, 16
    B = torch.arange(2 * out * r, dtype=torch.float32).reshape(2, out, r) + 1
    C = lora_b_chunk8(B)
    assert tuple(C.shape) == (2, 2, 8, 2, 64, 8)
    for a in range(2):
        for j in range(2):
            for i in range(8):
                for k in range(2):
                    for lane in range(64):
                        row = 8 * (64 * j + lane) + i
                        want = B[a, row, 8 * k: 8 * k + 8] if row < out else torch.zeros(8)
                        assert torch.equal(C[a, j, i, k, lane], want)
    with pytest.raises(ValueError):
        lora_b_chunk8(torch.zeros(2, 20, 16))
