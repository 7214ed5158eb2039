"""GPU test of the measurement-only streaming copy (ck_hbm_copy): exact
bytes for sizes around the grid-stride boundaries, nothing written past the
end."""

from __future__ import annotations

import pytest
import torch

from carrykernel_amd import _native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,grid", [(16, 0), (8192 * 3 + 16, 0), (1 << 20, 7), ((1 << 22) + 48, 0)])
def test_hbm_copy_exact(device, nbytes, grid):
    print(f"case hbm copy bytes={nbytes} grid={grid}", flush=True)
    g = torch.Generator(device=device).manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes + 64,), dtype=torch.uint8, generator=g, device=device)
    dst = torch.full((nbytes + 64,), 7, dtype=torch.uint8, device=device)
    _native.check(_native.lib().ck_hbm_copy(src.data_ptr(), dst.data_ptr(), nbytes, grid,
                                            _native.stream_handle(device)), "hbm copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src[:nbytes])
    assert torch.all(dst[nbytes:] == 7)
