"""The batched region copy (dnx_copy_regions): the commit's copy-backs to the
host views in one launch. Every byte of every region lands, nothing
around the regions is touched, and a pinned host destination is written
directly."""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D

pytestmark = pytest.mark.gpu


def test_copy_regions_device_and_pinned(gpu_ready):
    rng = np.random.default_rng(3)
    src = torch.from_numpy(rng.integers(0, 256, size=1 << 22, dtype=np.uint8)).cuda()
    dst_dev = torch.zeros(1 << 22, dtype=torch.uint8, device="cuda")
    dst_host = torch.zeros(1 << 22, dtype=torch.uint8).pin_memory()
    # (src offset, dst offset, bytes): aligned and misaligned, one byte,
    # several chunks, a region of zero bytes, a large one; destinations
    # disjoint (regions are copied concurrently).
    spec = [(0, 0, 16), (16, 64, 32768), (100001, 200003, 777), (5, 40, 1), (65536, 131072, 0),
            (1 << 20, 1 << 21, 608 * 1024), (3 << 20, 3 << 20, 16384 * 3 + 16)]
    regions = []
    for so, do, nb in spec:
        regions.append((src.data_ptr() + so, dst_dev.data_ptr() + do, nb))
        regions.append((src.data_ptr() + so, dst_host.data_ptr() + do, nb))
    D.copy_regions(regions)
    torch.cuda.synchronize()
    s = src.cpu().numpy()
    want = np.zeros(1 << 22, dtype=np.uint8)
    for so, do, nb in spec:
        want[do:do + nb] = s[so:so + nb]
    assert np.array_equal(dst_dev.cpu().numpy(), want)
    assert np.array_equal(dst_host.numpy(), want)


def test_copy_regions_limits(gpu_ready):
    t = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    D.copy_regions([])  # nothing to copy
    with pytest.raises(RuntimeError):
        D.copy_regions([(t.data_ptr(), t.data_ptr() + 2048, 16)] * 97)  # above DNX_COPY_MAX
    with pytest.raises(RuntimeError):
        D.copy_regions([(t.data_ptr(), t.data_ptr() + 2048, -1)])
