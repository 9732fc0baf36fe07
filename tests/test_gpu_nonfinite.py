"""Non-finite inputs: where an inf or NaN reaches, on the GPU.

The reference's loops never read a masked key (src/attention.zig:117-147,
every loop bounded by t + 1), so a non-finite value in K or V row s reaches
only the queries t >= s.  The kernels here remove a masked pair with a zero
weight or a -inf score instead (include/zt_attn.h, conventions), and these
tests pin exactly how far that differs:

  * scores are masked by a select, so a non-finite K row never reaches an
    earlier query: rows t < s are bit-identical to the finite run;
  * P = 0 times an infinite V entry is NaN, so a non-finite V row can reach
    the earlier queries that share its staged key tile, and only in that
    column: at most WINDOW rows before s, every other column bit-identical;
  * the queries the reference itself reaches get what the reference gives
    (+inf in that column, the CPU restatement agreeing);
  * cache rows past a sequence's n_keys are never read: NaN there changes no
    bit of any decode or forward result (a serving cache is not cleared).
"""
import numpy as np
import pytest

from gpuhelp import SEED_DO, SEED_K, SEED_KC, SEED_Q, SEED_V, SEED_VC, dev_normal, host

pytestmark = pytest.mark.gpu

B, T, H, Hkv, D = 1, 512, 8, 2, 64
GROUP = H // Hkv
BAD_S, BAD_KVH, BAD_D = 300, 1, 5
# The widest staged key tile (64 keys) plus the 16 rows of one MFMA tile.
WINDOW = 80


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _inputs(gpu, zt):
    q = dev_normal(gpu, zt, B * T * H * D, SEED_Q)
    k = dev_normal(gpu, zt, B * T * Hkv * D, SEED_K)
    v = dev_normal(gpu, zt, B * T * Hkv * D, SEED_V)
    do = dev_normal(gpu, zt, B * T * H * D, SEED_DO)
    return q, k, v, do


def _poke(t, row, kvh, col, value):
    """A copy of a [T, Hkv*D] tensor with one element replaced."""
    t = t.clone()
    t[row * Hkv * D + kvh * D + col] = value
    return t


def _forward(gpu, zt, path, q, k, v):
    out = gpu.full((B * T * H * D,), float("nan"), device="cuda")
    lse = gpu.empty(B * T * H, device="cuda")
    if path == "reference_abi":
        zt.forward(q, k, v, out, T, H, Hkv, D)
    elif path == "train":
        zt.forward_train(q, k, v, out, lse, T, H, Hkv, D)
    else:  # the scores-writing forward of the training step
        ws = gpu.empty(zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4, device="cuda")
        zt.forward_train_ws(q, k, v, out, lse, ws, T, H, Hkv, D)
    gpu.cuda.synchronize()
    return host(out).reshape(T, H, D)


@pytest.mark.parametrize("path", ["reference_abi", "train", "train_scores"])
def test_an_infinite_v_entry_reaches_only_its_column_and_key_tile(gpu, zt, oracle, path):
    q, k, v, _ = _inputs(gpu, zt)
    v_bad = _poke(v, BAD_S, BAD_KVH, BAD_D, float("inf"))
    good, bad = _forward(gpu, zt, path, q, k, v), _forward(gpu, zt, path, q, k, v_bad)
    hs = slice(BAD_KVH * GROUP, (BAD_KVH + 1) * GROUP)
    other = [h for h in range(H) if not BAD_KVH * GROUP <= h < (BAD_KVH + 1) * GROUP]
    # The other KV group, every column other than BAD_D, and the rows before the window: untouched.
    assert np.array_equal(_bits(bad[:, other]), _bits(good[:, other]))
    keep = np.ones(D, bool)
    keep[BAD_D] = False
    assert np.array_equal(_bits(bad[:, hs][:, :, keep]), _bits(good[:, hs][:, :, keep]))
    assert np.array_equal(_bits(bad[:BAD_S - WINDOW, hs]), _bits(good[:BAD_S - WINDOW, hs]))
    # Inside the window (t < s): the finite value, or NaN where 0 * inf was formed.
    win_bad, win_good = bad[BAD_S - WINDOW:BAD_S, hs, BAD_D], good[BAD_S - WINDOW:BAD_S, hs, BAD_D]
    assert np.all(np.isnan(win_bad) | (_bits(win_bad) == _bits(win_good)))
    # From row s on, what the reference gives: +inf in that column.
    assert np.all(np.isposinf(bad[BAD_S:, hs, BAD_D]))
    ref = oracle.attention_forward(host(q), host(k), host(v_bad), B, T, H, Hkv, D, t_begin=BAD_S,
                                   t_end=BAD_S + 16).reshape(-1, H, D)
    assert np.all(np.isposinf(ref[BAD_S:BAD_S + 16, hs, BAD_D]))


@pytest.mark.parametrize("path", ["reference_abi", "train", "train_scores"])
def test_a_non_finite_k_row_never_reaches_an_earlier_query(gpu, zt, path):
    q, k, v, _ = _inputs(gpu, zt)
    good = _forward(gpu, zt, path, q, k, v)
    for value in (float("inf"), float("nan")):
        bad = _forward(gpu, zt, path, q, _poke(k, BAD_S, BAD_KVH, BAD_D, value), v)
        assert np.array_equal(_bits(bad[:BAD_S]), _bits(good[:BAD_S])), value


def _backward(gpu, zt, path, q, k, v, do):
    dq = gpu.full((B * T * H * D,), float("nan"), device="cuda")
    dk, dv = (gpu.full((B * T * Hkv * D,), float("nan"), device="cuda") for _ in range(2))
    rows = [gpu.empty(B * T * H, device="cuda") for _ in range(3)]
    if path == "reference_abi":
        zt.backward(q, k, v, do, dq, dk, dv, *rows, T, H, Hkv, D)
    else:
        out = gpu.empty(B * T * H * D, device="cuda")
        lse, delta = rows[0], rows[1]
        if path == "train":
            zt.forward_train(q, k, v, out, lse, T, H, Hkv, D)
            zt.backward_train(q, k, v, out, do, lse, dq, dk, dv, delta, T, H, Hkv, D)
        else:
            ws = gpu.empty(zt.backward_train_workspace_bytes(B, T, H, Hkv, D) // 4, device="cuda")
            zt.forward_train_ws(q, k, v, out, lse, ws, T, H, Hkv, D)
            zt.backward_train_ws(q, k, v, out, do, lse, dq, dk, dv, ws, T, H, Hkv, D, stage=3 | zt.ZT_WS_SCORES)
    gpu.cuda.synchronize()
    return host(dq).reshape(T, H, D), host(dk).reshape(T, Hkv, D), host(dv).reshape(T, Hkv, D)


@pytest.mark.parametrize("path", ["reference_abi", "train", "train_scores"])
def test_an_infinite_v_entry_leaves_earlier_dq_rows_and_the_other_group_untouched(gpu, zt, path):
    """The reference's own gradients are non-finite for every row the bad
    entry reaches through O (t >= s) and for dk, dv of that KV head; the rows
    before the window and the other KV group stay bit-identical here."""
    q, k, v, do = _inputs(gpu, zt)
    good = _backward(gpu, zt, path, q, k, v, do)
    bad = _backward(gpu, zt, path, q, k, _poke(v, BAD_S, BAD_KVH, BAD_D, float("inf")), do)
    other = [h for h in range(H) if h // GROUP != BAD_KVH]
    assert np.array_equal(_bits(bad[0][:, other]), _bits(good[0][:, other]))
    assert np.array_equal(_bits(bad[0][:BAD_S - WINDOW]), _bits(good[0][:BAD_S - WINDOW]))
    for g_bad, g_good in zip(bad[1:], good[1:]):
        assert np.array_equal(_bits(g_bad[:, 1 - BAD_KVH]), _bits(g_good[:, 1 - BAD_KVH]))


def _decode_inputs(gpu, zt, Bd, n_ctx, Hd, Hkvd, Dd):
    q = dev_normal(gpu, zt, Bd * Hd * Dd, SEED_Q)
    kc = dev_normal(gpu, zt, Bd * n_ctx * Hkvd * Dd, SEED_KC)
    vc = dev_normal(gpu, zt, Bd * n_ctx * Hkvd * Dd, SEED_VC)
    return q, kc, vc


def _poison_past(t, n_keys, n_ctx, width):
    """A copy of a [B, n_ctx, width] cache with every row past each sequence's
    n_keys set to NaN, and its last row to -inf."""
    t = t.clone().view(len(n_keys), n_ctx, width)
    for b, nk in enumerate(n_keys):
        t[b, nk:] = float("nan")
        if nk < n_ctx:
            t[b, n_ctx - 1] = float("-inf")
    return t.view(-1)


@pytest.mark.parametrize("wgs", [None, "256", "32768"])
def test_decode_never_reads_cache_rows_past_n_keys(gpu, zt, tune, wgs):
    """One chunk per sequence, and split chunks (the workgroup target forced)."""
    if wgs:
        tune({"ZT_DEC_WGS": wgs})
    Bd, n_ctx, Hd, Hkvd, Dd = 6, 700, 32, 8, 128
    n_keys = [700, 699, 513, 64, 17, 1]
    q, kc, vc = _decode_inputs(gpu, zt, Bd, n_ctx, Hd, Hkvd, Dd)
    ws = gpu.empty(zt.decode_workspace_bytes(Bd, n_ctx, Hd, Hkvd, Dd) // 4 + 1, device="cuda")
    outs = []
    for kk, vv in ((kc, vc), (_poison_past(kc, n_keys, n_ctx, Hkvd * Dd), _poison_past(vc, n_keys, n_ctx, Hkvd * Dd))):
        out = gpu.full((Bd * Hd * Dd,), float("nan"), device="cuda")
        zt.decode(q, kk, vv, out, n_keys, Bd, n_ctx, Hd, Hkvd, Dd, ws)
        gpu.cuda.synchronize()
        outs.append(host(out))
    assert np.all(np.isfinite(outs[0]))
    assert np.array_equal(_bits(outs[1]), _bits(outs[0]))


@pytest.mark.parametrize("T_q,q_offset,n_keys", [(1, 299, 300), (1, 0, 1), (37, 263, 300), (64, 0, 64)])
def test_the_forward_never_reads_kv_rows_past_n_keys(gpu, zt, T_q, q_offset, n_keys):
    """zt_attn_forward_batched over caches of kv_rows > n_keys rows: the one-row
    route (T = 1, the reference decode seam) and the tiled kernels."""
    Bd, kv_rows, Hd, Hkvd, Dd = 3, 400, 8, 2, 128
    q = dev_normal(gpu, zt, Bd * T_q * Hd * Dd, SEED_Q)
    _, kc, vc = _decode_inputs(gpu, zt, Bd, kv_rows, Hd, Hkvd, Dd)
    nks = [n_keys] * Bd
    outs = []
    for kk, vv in ((kc, vc), (_poison_past(kc, nks, kv_rows, Hkvd * Dd), _poison_past(vc, nks, kv_rows, Hkvd * Dd))):
        out = gpu.full((Bd * T_q * Hd * Dd,), float("nan"), device="cuda")
        zt.forward(q, kk, vv, out, T_q, Hd, Hkvd, Dd, q_offset=q_offset, n_keys=n_keys, B=Bd, kv_rows=kv_rows)
        gpu.cuda.synchronize()
        outs.append(host(out))
    assert np.all(np.isfinite(outs[0]))
    assert np.array_equal(_bits(outs[1]), _bits(outs[0]))


def test_decode_propagates_a_visible_infinite_v_entry_as_the_reference(gpu, zt, oracle):
    Bd, n_ctx, Hd, Hkvd, Dd = 2, 300, 8, 2, 64
    n_keys = [300, 200]
    q, kc, vc = _decode_inputs(gpu, zt, Bd, n_ctx, Hd, Hkvd, Dd)
    ws = gpu.empty(zt.decode_workspace_bytes(Bd, n_ctx, Hd, Hkvd, Dd) // 4 + 1, device="cuda")
    vb = vc.clone().view(Bd, n_ctx, Hkvd, Dd)
    vb[0, 150, 1, 7] = float("inf")   # visible to sequence 0
    vb[1, 250, 1, 7] = float("inf")   # past sequence 1's n_keys
    vb = vb.view(-1)
    out = gpu.full((Bd * Hd * Dd,), float("nan"), device="cuda")
    zt.decode(q, kc, vb, out, n_keys, Bd, n_ctx, Hd, Hkvd, Dd, ws)
    good = gpu.full((Bd * Hd * Dd,), float("nan"), device="cuda")
    zt.decode(q, kc, vc, good, n_keys, Bd, n_ctx, Hd, Hkvd, Dd, ws)
    gpu.cuda.synchronize()
    got, fin = host(out).reshape(Bd, Hd, Dd), host(good).reshape(Bd, Hd, Dd)
    ref = oracle.attn_step(host(q), host(kc), host(vb), n_keys, Bd, n_ctx, Hd, Hkvd, Dd).reshape(Bd, Hd, Dd)
    hs = slice(Hd // Hkvd, Hd)
    assert np.all(np.isposinf(got[0, hs, 7])) and np.all(np.isposinf(ref[0, hs, 7]))
    got[0, hs, 7] = fin[0, hs, 7]
    assert np.array_equal(_bits(got), _bits(fin))
