"""Shared helpers for the GPU parity tests (host-side comparison only)."""
import numpy as np
import torch


def to_dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def rms(y):
    y = np.asarray(y, np.float64)
    return float(np.sqrt(np.mean(y * y))) if y.size else 0.0


def assert_close_rms(got, ref, what, rel=1e-3, fp16_out=False):
    """north_star bound: max|got - ref| <= 1e-3 * RMS(ref). For an fp16 output the
    unavoidable storage rounding (half an fp16 ulp of each element) is added to the
    bound; the fp32-output run of the same kernel is held to the bare bound."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    bound = rel * rms(ref)
    if fp16_out:
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
        bound = bound + 0.5 * ulp
    bad = err > bound
    assert not bad.any(), (
        f"{what}: max|err|={err.max():.3e} rms={rms(ref):.3e} "
        f"(bound {rel}*rms{'+ulp/2' if fp16_out else ''}) at {np.argwhere(bad)[:3].tolist()}")
    return float(err.max() / max(rms(ref), 1e-30))
