"""Helpers for the GPU parity tests: numpy <-> device tensors and the float tolerance."""
import numpy as np

# Float tolerance of the verify-step parity bar: relative to the norm, and absolute.
REL_NORM_TOL = 2e-2
ABS_TOL = 1e-2


def dev(a):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a.copy()).cuda()


def host(t, dtype=None):
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def close_report(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = float(np.abs(got - ref).max()) if got.size else 0.0
    return rel, mx


def assert_close(got, ref, rel_tol=REL_NORM_TOL, abs_tol=ABS_TOL, what=""):
    rel, mx = close_report(got, ref)
    print(f"[{what}] rel_norm={rel:.3e} max_abs={mx:.3e}", flush=True)
    if not (rel <= rel_tol and mx <= abs_tol) and np.ndim(got) == 2:
        # which rows and columns are off, to tell a wrong row from scattered noise
        d = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
        bad = d > abs_tol
        print(f"[{what}] rows off: {np.nonzero(bad.any(axis=1))[0].tolist()}; columns off per "
              f"row: {bad.sum(axis=1).tolist()}", flush=True)
    assert rel <= rel_tol and mx <= abs_tol, (what, rel, mx)
    return rel, mx
