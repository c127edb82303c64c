"""Child process of tests/test_gpu_forward.py: the same small decoder pass
with the environment the parent sets (DIANOIA_GPU_TRACK_WRITES=0); writes
its logits and upload bytes to gpurun_out/forward_child.npz."""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import numpy as np  # noqa: E402

from dianoia_amd import forward as F  # noqa: E402
from test_gpu_forward import qwen3_small, run  # noqa: E402


def main():
    fwd = F.GpuForward(qwen3_small(), max_seq=64, max_chunk=8, seed=9)
    run(fwd, [(8, 0), (8, 8), (1, 16)])
    logits16 = fwd.logits.copy()
    up0, _ = F.transfer_bytes()
    run(fwd, [(1, 17)])
    up17 = F.transfer_bytes()[0] - up0
    logits17 = fwd.logits.copy()
    fwd.dispose()
    os.makedirs(os.path.join(ROOT, "gpurun_out"), exist_ok=True)
    np.savez(os.path.join(ROOT, "gpurun_out", "forward_child.npz"), logits16=logits16,
             logits17=logits17, up17=up17, tracking=int(F.tracking_writes()))


if __name__ == "__main__":
    main()
