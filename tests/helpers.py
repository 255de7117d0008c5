"""Shared test helpers: tolerance metrics, host<->device copies."""
import numpy as np

MAX_REL = 1e-2
MIN_COS = 0.9999


def metrics(got, ref):
    """Normwise max relative error max|g-r|/max|r| and cosine similarity."""
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    denom = max(np.abs(r).max(), 1e-30)
    rel = float(np.abs(g - r).max() / denom)
    nrm = np.sqrt((g * g).sum() * (r * r).sum())
    cos = float((g * r).sum() / nrm) if nrm > 0 else (1.0 if np.abs(g).max() == 0 else 0.0)
    return rel, cos


def assert_close(got, ref, what=""):
    rel, cos = metrics(got, ref)
    assert rel <= MAX_REL and cos >= MIN_COS, f"{what}: max_rel={rel:.3e} cos={cos:.6f}"
    return rel, cos


def to_dev(a):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def to_host(t):
    import torch

    t = t.detach()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.cpu().numpy().view(np.uint32)
    return t.cpu().numpy()
