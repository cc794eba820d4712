"""The HBM read-floor probe (va_hbm_read_probe) that bench.py's floor leg times."""

import pytest
import torch

from voiceagent_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,wgs", [(16, 1), (46_373_936, 256), (1 << 20, 2048),
                                        (4096 * 16 + 16, 7)])
def test_probe_reads_without_writing(dev, nbytes, wgs):
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(wgs, dtype=torch.int32, device=dev)
    ops.hbm_read_probe(buf, wgs, sink)
    torch.cuda.synchronize()
    assert torch.count_nonzero(sink).item() == 0  # the fold of zeros never matches


def test_probe_rejects_unaligned_sizes(dev):
    buf = torch.zeros(40, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    with pytest.raises(ops.AttentionArgumentError):
        ops.hbm_read_probe(buf[:20], 1, sink)
    with pytest.raises(ops.AttentionArgumentError):
        ops.hbm_read_probe(buf[:32], 8, sink)
