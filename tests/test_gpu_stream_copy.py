"""hydra_stream_copy, the same-device copy bench.py times as the HBM ceiling
of one-pass kernels: bit-exact at ragged and full sizes."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, 3 * 256 * 16 + 48, 25_427_968])
def test_stream_copy_bit_exact(cuda, nbytes):
    from hydra_amd import _lib

    g = torch.Generator(device=cuda).manual_seed(nbytes % 1000)
    src = torch.randint(0, 256, (nbytes + 64,), device=cuda, dtype=torch.uint8, generator=g)
    dst = torch.zeros(nbytes + 64, device=cuda, dtype=torch.uint8)
    _lib.call("hydra_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, _lib.stream(src))
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src[:nbytes])
    assert not dst[nbytes:].any()  # nothing written past the range
