"""BatchFetcher on the GPU, streamed from the host and device-resident:
every batch equals the host rows the reference's seeding selects
(oracle.batch_rows), in order, for random and consecutive rows, several
dtypes and row shapes; fetchers over parallel arrays draw the same rows
whichever way each runs; a fetcher can be closed while batches are in
flight."""

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("resident", [True, False])
@pytest.mark.parametrize("shuffle", [True, False])
def test_batches_match_rows(dev, shuffle, resident):
    import torch

    import sdfoam_amd

    n, B = 10_007, 1000
    data = torch.arange(n * 6, dtype=torch.float32).reshape(n, 6)
    f = sdfoam_amd.BatchFetcher(data, B, shuffle=shuffle, resident=resident)
    assert f.resident == resident
    for b in range(12):  # three trips around the 4-slot ring
        got = f.next()
        assert got.shape == (B, 6) and got.device.type == "cuda" and got.dtype == torch.float32
        want = data.numpy()[oracle.batch_rows(b, B, n, shuffle)]
        assert np.array_equal(got.cpu().numpy(), want), f"batch {b}"
    f.close()


def test_parallel_arrays_draw_the_same_rows(dev):
    import torch

    import sdfoam_amd

    n, B = 5000, 777
    rays = torch.randn(n, 2, 3)
    ids = torch.arange(n, dtype=torch.int64).reshape(n, 1)
    tags = (torch.arange(n) % 251).to(torch.uint8).reshape(n, 1)
    fr = sdfoam_amd.BatchFetcher(rays, B, shuffle=True)
    fi = sdfoam_amd.BatchFetcher(ids, B, shuffle=True, resident=False)
    ft = sdfoam_amd.BatchFetcher(tags, B, shuffle=True)
    # whole-word rows go device-resident by default, byte rows are streamed;
    # the ids are streamed on request
    assert fr.resident and not fi.resident and not ft.resident
    for b in range(5):
        r, i, t = fr.next(), fi.next(), ft.next()
        rows = i.cpu().numpy().reshape(-1)
        assert np.array_equal(rows, oracle.batch_rows(b, B, n, True).astype(np.int64))
        assert torch.equal(r.cpu(), rays[rows])
        assert torch.equal(t.cpu(), tags[rows])
    for f in (fr, fi, ft):
        f.close()


@pytest.mark.parametrize("resident", [True, False])
def test_large_batches_and_early_close(dev, resident):
    """2^18 rows of 24 bytes from a 1M-row array (gathered by several
    threads, or by the GPU), consumed on a side stream; then closed with
    uploads pending."""
    import torch

    import sdfoam_amd

    n, B = 1_000_000, 1 << 18
    data = torch.randn(n, 6)
    f = sdfoam_amd.BatchFetcher(data, B, shuffle=True, resident=resident)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        outs = [f.next() for _ in range(3)]
    s.synchronize()
    for b, o in enumerate(outs):
        assert torch.equal(o.cpu(), data[oracle.batch_rows(b, B, n, True).astype(np.int64)])
    f.close()
    with pytest.raises(RuntimeError, match="closed"):
        f.next()


def test_rejects_cuda_data(dev):
    import torch

    import sdfoam_amd

    with pytest.raises(RuntimeError, match="CPU tensor"):
        sdfoam_amd.BatchFetcher(torch.zeros(10, 3, device=dev), 4, shuffle=True)


def test_resident_needs_whole_words(dev):
    import torch

    import sdfoam_amd

    with pytest.raises(RuntimeError, match="whole 32-bit words"):
        sdfoam_amd.BatchFetcher(torch.zeros(10, 3, dtype=torch.uint8), 4, shuffle=True,
                                resident=True)
