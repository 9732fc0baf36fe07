"""Pins the CPU restatement (oracle/) before anything is graded against it.

Each oracle function is checked against (a) the reference's own known-answer
tests (tests/golden/reference_known_answers.json), (b) an independent float64
numpy formulation (tests/npref.py) on random shapes, (c) finite differences
for the backward, and (d) closed forms and invariants the mathematics fixes.
The reference itself (Zig 0.16 + CUDA) cannot be built in this image.
"""
import numpy as np
import pytest

from npref import attention_backward_f64, attention_f64, attention_loss_grads_fd


def _rand(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- forward --

def test_forward_reference_known_answers(oracle, golden):
    for case in golden["attention"]:
        out = oracle.attention_forward(case["q"], case["k"], case["v"], 1, case["T"], case["H"], case["Hkv"],
                                       case["D"])
        want = np.asarray(case["out"], np.float32)
        if case["tol"] is None:
            assert np.array_equal(out, want), case["name"]
        else:
            assert np.max(np.abs(out - want)) <= case["tol"], case["name"]


def test_forward_groups_query_heads_onto_kv_head(oracle, golden):
    c = golden["attention_gqa"]
    out = oracle.attention_forward(c["q"], c["k"], c["v"], 1, c["T"], c["H"], c["Hkv"], c["D"]).reshape(2, 8)
    assert np.array_equal(out[0, 0:2], np.float32(c["row0_head0"]))
    assert np.array_equal(out[0, 4:6], np.float32(c["row0_head2"]))
    for t in range(2):
        assert np.array_equal(out[t, 0:2], out[t, 2:4])
        assert out[t, 0] != out[t, 4]


def test_forward_is_causal(oracle, golden):
    c = golden["attention_causal"]
    k = np.float32(c["k"]).reshape(3, 2)
    v = np.float32(c["v"]).reshape(3, 2)
    before = oracle.attention_forward(c["q"], k, v, 1, 3, 2, 1, 2).reshape(3, 4)
    k[1] = c["edit"]["k_row1"]
    v[1] = c["edit"]["v_row1"]
    after = oracle.attention_forward(c["q"], k, v, 1, 3, 2, 1, 2).reshape(3, 4)
    assert np.array_equal(before[0].view(np.uint32), after[0].view(np.uint32))
    assert after[1, 0] != before[1, 0]


def test_forward_bit_reproducible(oracle, golden):
    c = golden["attention_reproducible"]
    a = oracle.attention_forward(c["q"], c["k"], c["v"], 1, c["T"], c["H"], c["Hkv"], c["D"])
    b = oracle.attention_forward(c["q"], c["k"], c["v"], 1, c["T"], c["H"], c["Hkv"], c["D"])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_forward_refuses_bad_head_config(oracle, golden):
    for H, Hkv, D in golden["attention_refusals"]["configs"]:
        with pytest.raises(oracle.OracleRefused):
            oracle.attention_forward(np.zeros(max(1, H * D)), np.zeros(max(1, Hkv * D)),
                                     np.zeros(max(1, Hkv * D)), 1, 1, H, Hkv, D)


def test_forward_zero_tokens(oracle):
    out = oracle.attention_forward(np.zeros(0), np.zeros(0), np.zeros(0), 1, 0, 1, 1, 2)
    assert out.size == 0


def test_forward_f64_context_512(oracle, golden):
    c = golden["attention_f64_context"]
    T, D = c["T"], c["D"]
    t, j = np.meshgrid(np.arange(T), np.arange(D), indexing="ij")
    x = np.where((t + j) % 2 == 0, np.float32(c["even"]), np.float32(c["odd"])).astype(np.float32)
    out = oracle.attention_forward(x, x, x, 1, T, 1, 1, D).reshape(T, D)
    ref = attention_f64(x, x, x, T, 1, 1, D)
    assert np.max(np.abs(out - ref) / np.abs(ref)) <= c["rel_tol"]


@pytest.mark.parametrize("T,H,Hkv,D", [(1, 1, 1, 2), (5, 4, 2, 8), (17, 6, 3, 12), (33, 8, 1, 32), (9, 2, 2, 64)])
def test_forward_matches_independent_f64(oracle, T, H, Hkv, D):
    rng = np.random.default_rng(T * 131 + H * 7 + D)
    q, k, v = _rand(rng, T, H * D), _rand(rng, T, Hkv * D), _rand(rng, T, Hkv * D)
    out = oracle.attention_forward(q, k, v, 1, T, H, Hkv, D).reshape(T, H * D)
    ref = attention_f64(q, k, v, T, H, Hkv, D)
    # f32 narrowing of an f64 result: within one f32 ulp of the f64 value.
    assert np.all(np.abs(out - ref) <= np.abs(ref) * 2 ** -23 + 1e-30)


def test_forward_row_subset_and_threads_are_bit_identical(oracle):
    rng = np.random.default_rng(3)
    B, T, H, Hkv, D = 2, 40, 4, 2, 16
    q, k, v = _rand(rng, B, T, H * D), _rand(rng, B, T, Hkv * D), _rand(rng, B, T, Hkv * D)
    full = oracle.attention_forward(q, k, v, B, T, H, Hkv, D).reshape(B, T, H * D)
    part = oracle.attention_forward(q, k, v, B, T, H, Hkv, D, t_begin=25, t_end=40).reshape(B, T, H * D)
    assert np.array_equal(full[:, 25:].view(np.uint32), part[:, 25:].view(np.uint32))
    mt = oracle.attention_forward(q, k, v, B, T, H, Hkv, D, threads=4).reshape(B, T, H * D)
    assert np.array_equal(full.view(np.uint32), mt.view(np.uint32))


def test_forward_at_offset_equals_the_rows_of_a_full_pass(oracle):
    # Query rows at positions q_offset.. over n_keys keys are the last rows of the
    # full causal pass over those keys (src/cuda/attn_kernels.cu:204-218).
    rng = np.random.default_rng(4)
    n_keys, T, H, Hkv, D = 30, 6, 4, 2, 8
    qa, k, v = _rand(rng, n_keys, H * D), _rand(rng, n_keys, Hkv * D), _rand(rng, n_keys, Hkv * D)
    full = oracle.attention_forward(qa, k, v, 1, n_keys, H, Hkv, D).reshape(n_keys, H * D)
    at = oracle.attention_forward_at(qa[n_keys - T:], k, v, 1, T, H, Hkv, D, n_keys - T, n_keys).reshape(T, H * D)
    assert np.array_equal(full[n_keys - T:].view(np.uint32), at.view(np.uint32))


# --------------------------------------------------------------- backward --

@pytest.mark.parametrize("T,H,Hkv,D", [(3, 2, 2, 4), (9, 4, 2, 12), (8, 4, 2, 32), (5, 6, 2, 8), (7, 3, 1, 6)])
def test_backward_matches_finite_differences(oracle, T, H, Hkv, D):
    rng = np.random.default_rng(100 + T + D)
    q, k, v, do = _rand(rng, T, H * D), _rand(rng, T, Hkv * D), _rand(rng, T, Hkv * D), _rand(rng, T, H * D)
    dq, dk, dv = oracle.attention_backward(q, k, v, do, 1, T, H, Hkv, D)
    fq, fk, fv = attention_loss_grads_fd(q, k, v, do, T, H, Hkv, D)
    for got, want in ((dq, fq), (dk, fk), (dv, fv)):
        assert np.max(np.abs(got - want)) <= 2e-6 * max(1.0, np.max(np.abs(want))), (T, H, Hkv, D)


@pytest.mark.parametrize("T,H,Hkv,D", [(20, 4, 2, 8), (33, 6, 3, 16), (16, 2, 1, 64)])
def test_backward_matches_matrix_form_f64(oracle, T, H, Hkv, D):
    rng = np.random.default_rng(200 + T)
    q, k, v, do = _rand(rng, T, H * D), _rand(rng, T, Hkv * D), _rand(rng, T, Hkv * D), _rand(rng, T, H * D)
    got = oracle.attention_backward(q, k, v, do, 1, T, H, Hkv, D)
    want = attention_backward_f64(q, k, v, do, T, H, Hkv, D)
    for g, w in zip(got, want):
        # dq is narrowed once; dk/dv carry one f32 rounding per accumulated term.
        assert np.max(np.abs(g - w)) <= 1e-5 * max(1.0, np.max(np.abs(w)))
    for variant in ("suffix_to_prefix", "no_jacobian", "no_scale"):
        bad = attention_backward_f64(q, k, v, do, T, H, Hkv, D, variant)
        assert max(np.max(np.abs(g - b)) for g, b in zip(got, bad)) > 1e-3, variant


def test_backward_closed_forms(oracle):
    # One key: p = 1, dp - delta = 0 exactly, so dq = dk = 0 and dv = sum_h dO.
    rng = np.random.default_rng(5)
    H, Hkv, D = 4, 2, 8
    q, k, v, do = _rand(rng, 1, H * D), _rand(rng, 1, Hkv * D), _rand(rng, 1, Hkv * D), _rand(rng, 1, H * D)
    dq, dk, dv = oracle.attention_backward(q, k, v, do, 1, 1, H, Hkv, D)
    assert np.all(dq == 0) and np.all(dk == 0)
    dor = do.reshape(H, D)
    assert np.allclose(dv.reshape(Hkv, D), dor[0::2] + dor[1::2], rtol=0, atol=1e-6)


def test_backward_invariants(oracle):
    # sum_s dS[t, s] = 0 so sum_s dk[s] = 0; sum_s p[t, s] = 1 so
    # sum_s dv[s] = sum over the group's heads and all rows of dO.
    rng = np.random.default_rng(6)
    T, H, Hkv, D = 48, 8, 2, 16
    q, k, v, do = _rand(rng, T, H * D), _rand(rng, T, Hkv * D), _rand(rng, T, Hkv * D), _rand(rng, T, H * D)
    dq, dk, dv = oracle.attention_backward(q, k, v, do, 1, T, H, Hkv, D)
    dk3, dv3 = dk.reshape(T, Hkv, D), dv.reshape(T, Hkv, D)
    assert np.max(np.abs(dk3.sum(0))) <= 1e-4 * np.abs(dk3).sum(0).max()
    want = do.reshape(T, Hkv, H // Hkv, D).sum(axis=(0, 2))
    assert np.allclose(dv3.sum(0), want, rtol=1e-5, atol=1e-4)


def test_backward_row_subset_and_threads_are_bit_identical(oracle):
    rng = np.random.default_rng(7)
    B, T, H, Hkv, D = 2, 30, 4, 2, 8
    q, k, v, do = (_rand(rng, B, T, H * D), _rand(rng, B, T, Hkv * D), _rand(rng, B, T, Hkv * D),
                   _rand(rng, B, T, H * D))
    dq, dk, dv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D)
    pq, pk, pv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, t_begin=20)
    qs = (B, T, H * D)
    ks = (B, T, Hkv * D)
    assert np.array_equal(dq.reshape(qs)[:, 20:], pq.reshape(qs)[:, 20:])
    assert np.array_equal(dk.reshape(ks)[:, 20:], pk.reshape(ks)[:, 20:])
    assert np.array_equal(dv.reshape(ks)[:, 20:], pv.reshape(ks)[:, 20:])
    mq, mk, mv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D, threads=3)
    assert np.array_equal(dq, mq) and np.array_equal(dk, mk) and np.array_equal(dv, mv)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("B,T,H,Hkv,D,kv0,kv1", [(2, 70, 8, 2, 32, 0, 1), (2, 70, 8, 2, 32, 1, 2),
                                                 (1, 45, 6, 3, 34, 0, 3), (1, 33, 4, 4, 16, 2, 3),
                                                 (1, 9, 2, 1, 8, 0, 1)])
def test_group_backward_is_bit_identical_to_the_serial_restatement(oracle, B, T, H, Hkv, D, kv0, kv1):
    """The two-phase parallel backward over whole kv groups gives every dq, dk
    and dv bit of the serial h -> t -> s restatement on those groups and
    leaves the rest zero (T not a multiple of the 8-row key blocks, 1-4 heads
    per group, several threads)."""
    rng = np.random.default_rng(B * 1000 + T)
    q, k, v, do = (_rand(rng, B, T, H * D), _rand(rng, B, T, Hkv * D), _rand(rng, B, T, Hkv * D),
                   _rand(rng, B, T, H * D))
    dq, dk, dv = oracle.attention_backward(q, k, v, do, B, T, H, Hkv, D)
    gq, gk, gv = oracle.attention_backward_groups(q, k, v, do, B, T, H, Hkv, D, kv0, kv1, threads=5)
    g = H // Hkv
    hq, hk = slice(kv0 * g, kv1 * g), slice(kv0, kv1)
    q4, gq4 = dq.reshape(B, T, H, D), gq.reshape(B, T, H, D)
    assert np.array_equal(_bits(q4[:, :, hq]), _bits(gq4[:, :, hq]))
    for ref, got in ((dk, gk), (dv, gv)):
        r4, g4 = ref.reshape(B, T, Hkv, D), got.reshape(B, T, Hkv, D)
        assert np.array_equal(_bits(r4[:, :, hk]), _bits(g4[:, :, hk]))
        rest = np.ones(Hkv, bool)
        rest[hk] = False
        assert not np.any(g4[:, :, rest])
    rest = np.ones(H, bool)
    rest[hq] = False
    assert not np.any(gq4[:, :, rest])


def test_group_backward_keeps_the_f32_read_modify_write_order(oracle):
    """What the bit-identity above rests on: at this size the f32 chain of dk
    / dv terms differs from the same terms summed in f64 and rounded once, so
    a group backward that reordered or widened the chain would not match."""
    from npref import attention_backward_f64
    rng = np.random.default_rng(3)
    B, T, H, Hkv, D = 1, 64, 4, 2, 32
    q, k, v, do = (_rand(rng, B, T, H * D), _rand(rng, B, T, Hkv * D), _rand(rng, B, T, Hkv * D),
                   _rand(rng, B, T, H * D))
    _, gk, gv = oracle.attention_backward_groups(q, k, v, do, B, T, H, Hkv, D, 0, Hkv, threads=4)
    _, fk, fv = attention_backward_f64(q, k, v, do, T, H, Hkv, D)
    assert not np.array_equal(_bits(gk), _bits(np.float32(fk)))
    assert not np.array_equal(_bits(gv), _bits(np.float32(fv)))
    assert np.max(np.abs(gk - fk)) <= 1e-5 * np.abs(fk).max()


@pytest.mark.parametrize("B,T,H,Hkv,D,kv0,kv1", [(2, 70, 8, 2, 32, 1, 2), (1, 45, 6, 3, 34, 0, 3)])
def test_group_forward_is_bit_identical_to_the_serial_restatement(oracle, B, T, H, Hkv, D, kv0, kv1):
    rng = np.random.default_rng(T)
    q, k, v = _rand(rng, B, T, H * D), _rand(rng, B, T, Hkv * D), _rand(rng, B, T, Hkv * D)
    ref = oracle.attention_forward(q, k, v, B, T, H, Hkv, D).reshape(B, T, H, D)
    got = oracle.attention_forward_groups(q, k, v, B, T, H, Hkv, D, kv0, kv1, threads=3).reshape(B, T, H, D)
    g = H // Hkv
    assert np.array_equal(_bits(ref[:, :, kv0 * g:kv1 * g]), _bits(got[:, :, kv0 * g:kv1 * g]))
    assert not np.any(got[:, :, :kv0 * g]) and not np.any(got[:, :, kv1 * g:])


def test_row_stats_match_forward_identity(oracle):
    # delta = sum_s p dp = dO . O, the identity the device backward relies on.
    rng = np.random.default_rng(8)
    T, H, Hkv, D = 20, 4, 2, 8
    q, k, v, do = _rand(rng, T, H * D), _rand(rng, T, Hkv * D), _rand(rng, T, Hkv * D), _rand(rng, T, H * D)
    m, l, d = oracle.attention_row_stats(q, k, v, do, 1, T, H, Hkv, D)
    o = attention_f64(q, k, v, T, H, Hkv, D).reshape(T, H, D)
    assert np.allclose(d.reshape(T, H), (o * do.reshape(T, H, D)).sum(-1), rtol=1e-9, atol=1e-12)
    s = np.einsum("thd,shd->hts", q.reshape(T, H, D).astype(np.float64),
                  np.repeat(k.reshape(T, Hkv, D), H // Hkv, axis=1).astype(np.float64)) / np.sqrt(D)
    s = np.where(np.tril(np.ones((T, T), bool))[None], s, -np.inf)
    assert np.allclose(m.reshape(T, H), s.max(-1).T, rtol=1e-12, atol=1e-12)
    assert np.allclose(l.reshape(T, H), np.exp(s - s.max(-1, keepdims=True)).sum(-1).T, rtol=1e-12)


# ----------------------------------------------------------------- decode --

def test_attn_step_is_the_last_row_of_a_full_pass(oracle):
    rng = np.random.default_rng(9)
    n_ctx, H, Hkv, D, B = 24, 4, 2, 8, 3
    kc, vc = _rand(rng, B, n_ctx, Hkv * D), _rand(rng, B, n_ctx, Hkv * D)
    qrows = _rand(rng, B, n_ctx, H * D)
    n_keys = np.array([1, 13, 24], np.int32)
    q = np.stack([qrows[b, n_keys[b] - 1] for b in range(B)])
    out = oracle.attn_step(q, kc, vc, n_keys, B, n_ctx, H, Hkv, D).reshape(B, H * D)
    for b in range(B):
        nk = int(n_keys[b])
        full = oracle.attention_forward(qrows[b, :nk], kc[b, :nk], vc[b, :nk], 1, nk, H, Hkv, D).reshape(nk, H * D)
        assert np.array_equal(full[nk - 1].view(np.uint32), out[b].view(np.uint32))


def test_attn_step_refuses(oracle):
    z = np.zeros(64, np.float32)
    with pytest.raises(oracle.OracleRefused):
        oracle.attn_step(z, z, z, [0], 1, 4, 2, 1, 8)   # empty prefix (decode.zig:350)
    with pytest.raises(oracle.OracleRefused):
        oracle.attn_step(z, z, z, [5], 1, 4, 2, 1, 8)   # beyond the cache
    with pytest.raises(oracle.OracleRefused):
        oracle.attn_step(z, z, z, [1], 1, 4, 3, 2, 8)   # 3 over 2 is not a group


# ---------------------------------------------------------------- rmsnorm --

def test_rmsnorm_reference_known_answers(oracle, golden):
    for c in golden["rmsnorm"]:
        y = oracle.rmsnorm(c["x"], c["w"], c["rows"], c["cols"])
        want = np.float32(c["y"])
        if c["tol"] is None:
            assert np.array_equal(y, want)
        else:
            assert np.max(np.abs(y - want)) <= c["tol"], c["src"]


def test_rmsnorm_f64_accumulator_over_512(oracle, golden):
    c = golden["rmsnorm_f64_row"]
    x = np.full(c["cols"], np.float32(c["x"]), np.float32)
    y = oracle.rmsnorm(x, np.ones(c["cols"], np.float32), 1, c["cols"])
    assert np.all(np.abs(y - np.float32(c["y_f32"])) <= c["tol"])
    assert abs(float(y[0]) - c["exact"]) <= c["tol"]
    # The same row summed in f32 lands outside the tolerance (norm_test.zig:93-138),
    # so this case does discriminate the accumulator width.
    s32 = np.float32(0)
    for _ in range(c["cols"]):
        s32 = np.float32(s32 + np.float32(c["x"]) * np.float32(c["x"]))
    rms32 = np.float32(np.sqrt(np.float64(s32) / c["cols"] + 1e-5))
    assert abs(np.float64(np.float32(c["x"])) / np.float64(rms32) - c["exact"]) > c["tol"]


def test_rmsnorm_constant_rows_closed_form(oracle):
    cols = 100
    vals = np.array([0.5, -3.0, 1e-3, 7.25], np.float32)
    x = np.repeat(vals, cols).astype(np.float32)
    w = np.linspace(0.5, 1.5, cols).astype(np.float32)
    y = oracle.rmsnorm(x, w, len(vals), cols).reshape(len(vals), cols)
    want = vals[:, None].astype(np.float64) / np.sqrt(vals[:, None].astype(np.float64) ** 2 + 1e-5) * w
    assert np.allclose(y, want, rtol=3e-7, atol=0)


# ------------------------------------------------------------------- rope --

def test_rope_reference_known_answers(oracle, golden):
    theta = golden["rope_theta"]["theta"]
    for c in golden["rope"]:
        y = oracle.rope(c["x"], c["rows"], c["cols"], c["pos"], theta, c["head_dim"])
        want = np.float32(c["y"])
        if c["tol"] is None:
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
        else:
            assert np.max(np.abs(y - want)) <= c["tol"], c["src"]
    c = golden["rope_norm"]
    y = oracle.rope(c["x"], 1, c["cols"], c["pos"], theta, c["head_dim"])
    assert abs(np.linalg.norm(y.astype(np.float64)) - c["l2"]) <= c["tol"]
    for cols, hd in golden["rope_refusals"]["odd"]:
        with pytest.raises(oracle.OracleRefused):
            oracle.rope(np.ones(cols), 1, cols, 0, theta, hd)
    for cols, hd in golden["rope_refusals"]["mismatch"]:
        with pytest.raises(oracle.OracleRefused):
            oracle.rope(np.ones(cols), 1, cols, 0, theta, hd)


def _rotation_matrix(oracle, cols, pos, theta, head_dim):
    # Columns of R are rope applied to the basis vectors: with one non-zero
    # input, each output is a single f32-narrowed cos or sin, so R is exact to
    # f32 rounding and independent of how rope_backward is written.
    return np.stack([oracle.rope(np.eye(cols, dtype=np.float32)[j], 1, cols, pos, theta, head_dim)
                     for j in range(cols)], axis=1).astype(np.float64)


@pytest.mark.parametrize("cols,head_dim,pos", [(8, 8, 0), (8, 8, 3), (24, 8, 17), (64, 32, 1000), (12, 4, 9)])
def test_rope_backward_is_the_transpose_of_rope(oracle, cols, head_dim, pos):
    # src/autograd.zig:851-872: din = R^T dout, R the rotation rope applies.
    theta = 500000.0
    R = _rotation_matrix(oracle, cols, pos, theta, head_dim)
    rng = np.random.default_rng(cols * 100 + pos)
    y = _rand(rng, cols)
    din = oracle.rope_backward(y, 1, cols, pos, theta, head_dim).astype(np.float64)
    assert np.max(np.abs(din - R.T @ y.astype(np.float64))) <= 2e-6
    if pos > 0:  # the forward rotation itself is not the answer (a sign slip would be)
        assert np.max(np.abs(din - R @ y.astype(np.float64))) > 1e-3
    # R orthogonal: backward undoes forward up to two f32 roundings.
    x = _rand(rng, cols)
    back = oracle.rope_backward(oracle.rope(x, 1, cols, pos, theta, head_dim), 1, cols, pos, theta, head_dim)
    assert np.max(np.abs(back - x)) <= 1e-6


def test_rope_backward_rows_advance_the_position(oracle):
    rows, cols, hd, theta = 5, 16, 8, 10000.0
    rng = np.random.default_rng(7)
    dout = _rand(rng, rows, cols)
    din = oracle.rope_backward(dout, rows, cols, 4, theta, hd).reshape(rows, cols)
    for r in range(rows):
        one = oracle.rope_backward(dout[r], 1, cols, 4 + r, theta, hd)
        assert np.array_equal(din[r], one)
    # Position 0: every angle is 0, so the gradient passes through unchanged.
    assert np.array_equal(oracle.rope_backward(dout[0], 1, cols, 0, theta, hd), dout[0])


def test_rope_backward_refusals(oracle):
    with pytest.raises(oracle.OracleRefused):
        oracle.rope_backward(np.ones(6), 1, 6, 0, 5e5, 3)
    with pytest.raises(oracle.OracleRefused):
        oracle.rope_backward(np.ones(6), 1, 6, 0, 5e5, 4)


# ------------------------------------------------------------ decode step --

@pytest.mark.parametrize("B,T,H,Hkv,D", [(2, 12, 4, 2, 32), (1, 9, 6, 3, 34), (3, 5, 2, 1, 64)])
def test_decode_step_sequence_equals_the_causal_forward(oracle, B, T, H, Hkv, D):
    # src/decode_test.zig:222-330: decoding a sequence token by token through a
    # filling cache agrees with the full causal forward over rotated q and k.
    theta = 500000.0
    rng = np.random.default_rng(B * 100 + T)
    q, k, v = _rand(rng, B, T, H * D), _rand(rng, B, T, Hkv * D), _rand(rng, B, T, Hkv * D)
    kc = np.zeros((B, T, Hkv * D), np.float32)
    vc = np.zeros((B, T, Hkv * D), np.float32)
    outs = []
    for t in range(T):
        out, kc, vc = oracle.decode_step(q[:, t], k[:, t], v[:, t], kc, vc, [t] * B, B, T, H, Hkv, D, theta)
        outs.append(out.reshape(B, H * D))
    dec = np.stack(outs, axis=1)
    qr = np.stack([oracle.rope(q[b], T, H * D, 0, theta, D) for b in range(B)])
    kr = np.stack([oracle.rope(k[b], T, Hkv * D, 0, theta, D) for b in range(B)])
    full = oracle.attention_forward(qr, kr, v, B, T, H, Hkv, D).reshape(B, T, H * D)
    assert np.max(np.abs(dec - full)) <= 1e-5
    assert np.array_equal(kc.reshape(B, T, -1), kr.reshape(B, T, -1))
    assert np.array_equal(vc.reshape(B, T, -1), v)
    # Unrotated keys would not agree: the check sees a missed rotation.
    wrong = oracle.attention_forward(qr, k, v, B, T, H, Hkv, D).reshape(B, T, H * D)
    assert np.max(np.abs(dec - wrong)) > 1e-3


def test_decode_step_refuses_a_full_cache(oracle):
    z = np.zeros(64, np.float32)
    with pytest.raises(oracle.OracleRefused):
        oracle.decode_step(z[:64], z[:32], z[:32], np.zeros(4 * 32), np.zeros(4 * 32), [4], 1, 4, 2, 1, 32)
    with pytest.raises(oracle.OracleRefused):
        oracle.decode_step(z[:64], z[:32], z[:32], np.zeros(4 * 32), np.zeros(4 * 32), [-1], 1, 4, 2, 1, 32)


# ------------------------------------------------------------- generators --

def test_generators_are_seeded_and_well_formed(oracle):
    a = oracle.fill_normal(200_000, 0x5EED0001)
    b = oracle.fill_normal(200_000, 0x5EED0001)
    c = oracle.fill_normal(1000, 0x5EED0001)
    assert np.array_equal(a, b) and np.array_equal(a[:1000], c)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    s2 = oracle.fill_normal(200_000, 0x5EED0002, 0.0, np.sqrt(2.0))
    assert abs(s2.var() - 2.0) < 0.03
    u = oracle.fill_uniform(100_000, 0x5EED0008, 0.5, 1.5)
    assert u.min() >= 0.5 and u.max() < 1.5 and abs(u.mean() - 1.0) < 0.01
    # splitmix64 known value (seed 0, first output), Vigna's reference generator.
    assert oracle.splitmix64(0, 0) == 0xE220A8397B1DCDAF


# ------------------------------------------------------------------ matmul --

def test_matmul_reference_known_answers(oracle, golden):
    for c in golden["matmul"]:
        got = oracle.matmul(c["a"], c["b"], c["M"], c["K"], c["N"])
        assert np.array_equal(got, np.float32(c["out"])), c["src"]


def _f32_gate(got, a, b, M, K, N):
    """The reference's accumulator-width statistic (src/tensor_test.zig:185-273):
    worst |got - f32(exact)| / sum|products|."""
    a64, b64 = a.reshape(M, K).astype(np.float64), b.reshape(K, N).astype(np.float64)
    exact = a64 @ b64
    abs_sum = np.abs(a64) @ np.abs(b64)
    wide = exact.astype(np.float32).astype(np.float64)
    return float(np.max(np.abs(got.reshape(M, N).astype(np.float64) - wide) / abs_sum))


def test_matmul_reduces_in_f32_not_f64(oracle, golden):
    c = golden["matmul_f32_gate"]
    M, K, N = c["M"], c["K"], c["N"]
    rng = np.random.default_rng(7)
    a = rng.uniform(c["lo"], c["hi"], M * K).astype(np.float32)
    b = rng.uniform(c["lo"], c["hi"], K * N).astype(np.float32)
    worst = _f32_gate(oracle.matmul(a, b, M, K, N), a, b, M, K, N)
    assert (K - 1) * np.finfo(np.float64).eps < worst < (K - 1) * np.finfo(np.float32).eps
    # A reduction carried in f64 (then stored in f32) sits on the f64 side of the gate.
    wide = (a.reshape(M, K).astype(np.float64) @ b.reshape(K, N)).astype(np.float32)
    assert _f32_gate(wide.ravel(), a, b, M, K, N) <= (K - 1) * np.finfo(np.float64).eps


@pytest.mark.parametrize("T,I,J", [(1, 1, 1), (7, 5, 9), (64, 24, 40), (300, 16, 8)])
def test_weight_and_input_grads_are_the_transposed_products(oracle, T, I, J):
    # weightGrad from zero is matmul(input^T, dout) and inputGrad from zero is
    # matmul(dout, w^T): the same products summed in the same order, so equal
    # bit for bit; a transposed operand or a swapped index fails.
    rng = np.random.default_rng(T * 100 + I)
    inp, dout = _rand(rng, T, I), _rand(rng, T, J)
    w = _rand(rng, I, J)
    wg = oracle.weight_grad(np.zeros(I * J), inp, dout, T, I, J)
    assert np.array_equal(wg, oracle.matmul(np.ascontiguousarray(inp.T), dout, I, T, J))
    ig = oracle.input_grad(np.zeros(T * I), dout, w, T, J, I)
    assert np.array_equal(ig, oracle.matmul(dout, np.ascontiguousarray(w.T), T, J, I))
    # Both accumulate onto what the buffer held (Tensor.init zeroes; blockBackward reuses).
    w0 = _rand(rng, I, J)
    wg2 = oracle.weight_grad(w0, inp, dout, T, I, J)
    want = w0.astype(np.float64).ravel() + (inp.astype(np.float64).T @ dout).ravel()
    assert np.max(np.abs(wg2 - want)) <= 1e-5 * max(1.0, np.abs(want).max())
    o0 = _rand(rng, T, I)
    ig2 = oracle.input_grad(o0, dout, w, T, J, I)
    want = o0.astype(np.float64).ravel() + (dout.astype(np.float64) @ w.T).ravel()
    assert np.max(np.abs(ig2 - want)) <= 1e-5 * max(1.0, np.abs(want).max())
