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
