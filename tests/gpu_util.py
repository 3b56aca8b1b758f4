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


def draft_q_values(rng, logits, draft, T):
    """Draft densities q_i as a suffix-tree draft source gives them (qAlong: child count over
    sibling mass, floored at 1e-6, 1 past the matched path), mixed with q = 0 (always rejected),
    and q near the target's own p on the draft (accept probability strictly inside (0, 1))."""
    q = np.empty(len(draft), np.float32)
    for i, d in enumerate(draft):
        l = logits[i].astype(np.float64) / T
        p = np.exp(l - l.max())
        pd = p[d] / p.sum()
        kind = int(rng.integers(0, 6))
        if kind == 0:
            q[i] = 0.0
        elif kind == 1:
            q[i] = 1e-6
        elif kind == 2:
            b = int(rng.integers(2, 8))
            q[i] = float(rng.integers(1, b + 1)) / b
        elif kind == 3:
            q[i] = min(1.0, pd * rng.uniform(0.4, 3.0))
        elif kind == 4:
            q[i] = 1.0
        else:
            q[i] = rng.uniform(0.0, 1.0)
    return q
