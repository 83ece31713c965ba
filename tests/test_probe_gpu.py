"""The measurement probes behind bench.py's measured ceilings (dk_probe_hbm, dk_probe_mfma_f16):
every variant of the HBM probe moves exactly the bytes it claims (a copy reproduces its source,
a fill writes its pattern), and the MFMA probe writes its output."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("units", [0, 16, 32])
@pytest.mark.parametrize("plain", [0, 4, 8, 12])
def test_hbm_probe_copy_and_fill(units, plain, device):
    from decik_amd import _lib

    L, stream = _lib.lib(), _lib.stream_of(device)
    n = (3 << 20) + 48  # bytes: not a multiple of any work-group's span (a partial last work-group)
    g = torch.Generator().manual_seed(units + plain)
    src = torch.randint(0, 1 << 30, (n // 4,), generator=g, dtype=torch.int32).to(device)
    dst = torch.zeros_like(src)
    sums = torch.zeros(n // 16384 + 1, dtype=torch.float32, device=device)
    _lib.check(L.dk_probe_hbm(src.data_ptr(), dst.data_ptr(), n, 2 + units + plain, sums.data_ptr(), stream))
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    _lib.check(L.dk_probe_hbm(src.data_ptr(), dst.data_ptr(), n, 1 + units + (plain & 4), sums.data_ptr(), stream))
    torch.cuda.synchronize()
    pattern = torch.tensor([0, 1, 2, 3], dtype=torch.int32, device=device)
    got = dst.view(-1, 4)
    assert torch.equal(got[:, 1:], pattern[1:].expand(got.shape[0], 3))
    assert set(got[:, 0].unique().tolist()) <= {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15}
    _lib.check(L.dk_probe_hbm(src.data_ptr(), dst.data_ptr(), n, units + (plain & 8), sums.data_ptr(), stream))
    torch.cuda.synchronize()


def test_mfma_probe_writes(device):
    from decik_amd import _lib

    L, stream = _lib.lib(), _lib.stream_of(device)
    out = torch.full((4 * 512,), float("nan"), dtype=torch.float32, device=device)
    _lib.check(L.dk_probe_mfma_f16(4, 8, out.data_ptr(), stream))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
