"""Helpers for the GPU parity tests: seeded device inputs (the library's own
fill kernel), copies back to the host, and the error measures the gates use."""
import numpy as np

# Seeds of the synthetic inputs: q, k, v, dO, cache K, cache V, norm x, gain.
SEED_Q, SEED_K, SEED_V, SEED_DO, SEED_KC, SEED_VC, SEED_X, SEED_W = (0x5EED0001 + i for i in range(8))
THETA = 500000.0

FWD_TOL = 1e-4    # max |out - twin|, forward and decode (north_star)
BWD_REL = 1e-3    # max |g - twin| / max |twin| per gradient (north_star)
BWD_FLOOR = 1e-6  # absolute floor, for gradients the twin makes exactly zero (dq, dk at T = 1)


def dev_normal(torch, zt, n, seed, sigma=1.0):
    t = torch.empty(n, device="cuda", dtype=torch.float32)
    zt.fill_normal(t, seed, 0.0, sigma)
    return t


def dev_uniform(torch, zt, n, seed, lo, hi):
    t = torch.empty(n, device="cuda", dtype=torch.float32)
    zt.fill_uniform(t, seed, lo, hi)
    return t


def host(t):
    return t.detach().cpu().numpy().ravel()


def max_abs(a, b):
    d = np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))
    d[~np.isfinite(d)] = np.inf   # a NaN or inf anywhere fails the gate
    return float(d.max()) if d.size else 0.0


def rel_err(a, b):
    """max|a - b| / max|b|, the reference's relative convention
    (src/train.zig:682-693), with BWD_FLOOR * BWD_REL^-1 as the smallest scale so
    a twin gradient that is exactly zero is met by rounding noise below 1e-6."""
    scale = float(np.max(np.abs(np.asarray(b, np.float64)))) if np.size(b) else 0.0
    return max_abs(a, b) / max(scale, BWD_FLOOR / BWD_REL)
