"""Independent float64 numpy formulation of causal GQA attention, used to pin
the oracle: whole-matrix products and a masked row softmax, a different
structure from the oracle's per-row loops, so an index, transpose or masking
slip in either shows up as a disagreement."""
import numpy as np


def attention_f64(q, k, v, T, H, Hkv, D, q_offset=0, n_keys=None):
    """q [T, H*D], k/v [n_keys, Hkv*D] -> out [T, H*D] in float64."""
    n_keys = T if n_keys is None else n_keys
    q = np.asarray(q, np.float64).reshape(T, H, D)
    k = np.asarray(k, np.float64).reshape(n_keys, Hkv, D)
    v = np.asarray(v, np.float64).reshape(n_keys, Hkv, D)
    g = H // Hkv
    out = np.zeros((T, H, D))
    vis = np.arange(n_keys)[None, :] <= (q_offset + np.arange(T))[:, None]
    for h in range(H):
        s = q[:, h, :] @ k[:, h // g, :].T / np.sqrt(D)
        s = np.where(vis, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ v[:, h // g, :]
    return out.reshape(T, H * D)


def attention_loss_grads_fd(q, k, v, dout, T, H, Hkv, D, eps=1e-6):
    """Central differences of L = sum(out * dout) in float64."""
    q = np.asarray(q, np.float64).ravel().copy()
    k = np.asarray(k, np.float64).ravel().copy()
    v = np.asarray(v, np.float64).ravel().copy()
    dout = np.asarray(dout, np.float64).ravel()

    def loss():
        return float(np.sum(attention_f64(q, k, v, T, H, Hkv, D).ravel() * dout))

    grads = []
    for x in (q, k, v):
        g = np.zeros_like(x)
        for i in range(x.size):
            old = x[i]
            x[i] = old + eps
            lp = loss()
            x[i] = old - eps
            lm = loss()
            x[i] = old
            g[i] = (lp - lm) / (2 * eps)
        grads.append(g)
    return grads


def attention_backward_f64(q, k, v, dout, T, H, Hkv, D, variant=None):
    """Matrix-form float64 backward (dq, dk, dv flat).  `variant` plants one of
    the reference's BROKEN backward defects (src/cuda/attn_kernels.cu:573-627):
      "suffix_to_prefix"  dk/dv summed over rows t <= s instead of t >= s
      "no_jacobian"       dS = P (dv unchanged)
      "no_scale"          scores and dq/dk without 1/sqrt(d)
      "gqa_collapsed"     every head reads and writes kv head 0"""
    q = np.asarray(q, np.float64).reshape(T, H, D)
    k = np.asarray(k, np.float64).reshape(T, Hkv, D)
    v = np.asarray(v, np.float64).reshape(T, Hkv, D)
    do = np.asarray(dout, np.float64).reshape(T, H, D)
    g = H // Hkv
    scale = 1.0 if variant == "no_scale" else 1.0 / np.sqrt(D)
    causal = np.tril(np.ones((T, T), bool))
    dq = np.zeros((T, H, D))
    dk = np.zeros((T, Hkv, D))
    dv = np.zeros((T, Hkv, D))
    for h in range(H):
        kv = 0 if variant == "gqa_collapsed" else h // g
        s = q[:, h] @ k[:, kv].T * scale
        sm = np.where(causal, s, -np.inf)
        m = sm.max(1, keepdims=True)
        l = np.exp(sm - m).sum(1, keepdims=True)
        p = np.exp(sm - m) / l
        dp = do[:, h] @ v[:, kv].T
        delta = (p * dp).sum(1, keepdims=True)
        ds = p if variant == "no_jacobian" else p * (dp - delta)
        dq[:, h] = ds @ k[:, kv] * scale
        if variant == "suffix_to_prefix":
            pw = np.where(causal.T, np.exp(s - m) / l, 0.0)
            dsw = pw * (dp - delta)
            dk[:, kv] += dsw.T @ q[:, h] * scale
            dv[:, kv] += pw.T @ do[:, h]
        else:
            dk[:, kv] += ds.T @ q[:, h] * scale
            dv[:, kv] += p.T @ do[:, h]
    return dq.ravel(), dk.ravel(), dv.ravel()
