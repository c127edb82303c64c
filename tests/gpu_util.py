"""Helpers shared by the GPU parity tests."""

import numpy as np


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def within_tolerance(gpu, cpu, rel=1e-4, abs_near_zero=1e-5):
    """The north-star bar for fp32 outputs: max relative error 1e-4, or
    absolute 1e-5 for values near zero. Returns (ok, worst_rel, worst_abs)."""
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    err = np.abs(gpu - cpu)
    ok = (err <= rel * np.abs(cpu)) | (err <= abs_near_zero)
    rel_err = np.where(np.abs(cpu) > 0, err / np.maximum(np.abs(cpu), 1e-30), err)
    return bool(ok.all()), float(rel_err[~(err <= abs_near_zero)].max(initial=0.0)), float(err.max(initial=0.0))
