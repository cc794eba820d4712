"""The HBM read-floor probe (va_bench_hbm_read in libvoiceagent_bench.so) that
bench.py's floor leg times, through each of its load paths."""

import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", sorted(bench.PROBE_MODES))
@pytest.mark.parametrize("nbytes,wgs", [(16, 1), (46_373_936, 256), (1 << 20, 2048),
                                        (4096 * 16 + 16, 7), (1040, 3)])
def test_probe_reads_without_writing(dev, mode, nbytes, wgs):
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(wgs, dtype=torch.int32, device=dev)
    print(f"probe mode={mode} bytes={nbytes} workgroups={wgs}", flush=True)
    bench.hbm_read(buf, wgs, mode, sink)
    torch.cuda.synchronize()
    assert torch.count_nonzero(sink).item() == 0  # the fold of zeros never matches


@pytest.mark.parametrize("rbytes,wbytes,wgs", [(1 << 20, 1 << 19, 256), (4096, 8192, 3),
                                               (70_131_712, 70_131_712, 2048)])
def test_copy_floor_writes_what_it_reads(dev, rbytes, wbytes, wgs):
    # va_bench_hbm_copy writes word j of the source where j < both counts,
    # and (j, 0, 0, 0) past the read count.
    g = torch.Generator(device=dev).manual_seed(5)
    src = torch.randint(0, 256, (rbytes,), dtype=torch.uint8, device=dev, generator=g)
    dst = torch.zeros(wbytes, dtype=torch.uint8, device=dev)
    print(f"copy floor read={rbytes} write={wbytes} workgroups={wgs}", flush=True)
    bench.hbm_copy(src, dst, wgs)
    torch.cuda.synchronize()
    n = min(rbytes, wbytes)
    assert torch.equal(dst[:n], src[:n])
    if wbytes > rbytes:
        words = dst[n:].view(torch.int32).view(-1, 4)
        j = torch.arange(n // 16, wbytes // 16, device=dev, dtype=torch.int32)
        assert torch.equal(words[:, 0], j) and torch.count_nonzero(words[:, 1:]).item() == 0


@pytest.mark.parametrize("wgs", [1, 256, 2048])
def test_empty_launch(dev, wgs):
    print(f"empty launch workgroups={wgs}", flush=True)
    bench.empty_launch(wgs)
    torch.cuda.synchronize()
