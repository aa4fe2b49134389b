"""pt_copy, the 16-byte streaming copy behind the benchmark's achievable-bandwidth line and
the counter calibration: every byte arrives, nothing past the end is written."""

from __future__ import annotations

import pytest
import torch

from picotron_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096, 4096 + 16, 255 * 16, 257 * 16, (1 << 20) + 48, 1 << 28])
def test_copy_moves_every_byte_and_nothing_more(gpu, nbytes):
    g = torch.Generator(device=gpu).manual_seed(nbytes % 9973)
    src = torch.randint(0, 256, (nbytes,), generator=g, device=gpu, dtype=torch.uint8)
    dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    ops.copy_bytes(src, dst[:nbytes])
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert bool((dst[nbytes:] == 0xA5).all())
