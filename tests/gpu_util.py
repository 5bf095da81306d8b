"""Helpers of the GPU tests: device upload and a one-line banner per GPU step (flushed, so a run that
dies names its case)."""
import sys

import numpy as np
import torch


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host_u16(t):
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.view(torch.int16)
    return t.cpu().numpy().view(np.uint16)


def banner(*args):
    print("[gpu-step]", *args, flush=True)
    sys.stdout.flush()


def close_rel(got, ref, rel=1e-3, floor=1e-4):
    """max over elements of |got - ref| / (rel |ref| + floor rms(row)) -- <= 1 passes."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True))
    tol = rel * np.abs(ref) + floor * rms
    return float(np.max(np.abs(got - ref) / np.maximum(tol, 1e-300)))
