"""Child process of tests/test_gpu_forward.py: the same small decoder pass
in a process of its own, writing its results as an .npz file to the
directory the parent names (the last argument).

* ``plain DIR``: with the environment the parent sets
  (DIANOIA_GPU_TRACK_WRITES=0); writes its logits and upload bytes to
  DIR/forward_child.npz;
* ``replace-handler DIR``: after a first pass with host-write tracking on,
  another SIGSEGV handler (the default action) replaces the library's; the
  next lab_gpu_contents must see that and turn tracking off, unprotecting
  every page, before the host writes again (a write to a still protected
  page would now end the process). Writes DIR/forward_child_handler.npz.
"""

import os
import signal
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import numpy as np  # noqa: E402

from dianoia_amd import forward as F  # noqa: E402
from test_gpu_forward import qwen3_small, run  # noqa: E402


def main(out_dir):
    fwd = F.GpuForward(qwen3_small(), max_seq=64, max_chunk=8, seed=9)
    run(fwd, [(8, 0), (8, 8), (1, 16)])
    logits16 = fwd.logits.copy()
    up0, _ = F.transfer_bytes()
    run(fwd, [(1, 17)])
    up17 = F.transfer_bytes()[0] - up0
    logits17 = fwd.logits.copy()
    fwd.dispose()
    np.savez(os.path.join(out_dir, "forward_child.npz"), logits16=logits16,
             logits17=logits17, up17=up17, tracking=int(F.tracking_writes()))


def replace_handler(out_dir):
    fwd = F.GpuForward(qwen3_small(), max_seq=64, max_chunk=8, seed=9)
    run(fwd, [(8, 0), (8, 8)])
    before = int(F.tracking_writes())
    signal.signal(signal.SIGSEGV, signal.SIG_DFL)
    fwd.residual  # a view: lab_gpu_contents
    after = int(F.tracking_writes())
    run(fwd, [(1, 16)])   # host writes into pages that were write-protected
    logits16 = fwd.logits.copy()
    fwd.dispose()
    np.savez(os.path.join(out_dir, "forward_child_handler.npz"), logits16=logits16,
             before=before, after=after)


if __name__ == "__main__":
    if sys.argv[1] == "replace-handler":
        replace_handler(sys.argv[2])
    else:
        main(sys.argv[2])
