"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle routine is checked against something independent of its own
formula:
  * the reference's own CPU routines, compiled from their source by
    oracle/build_ref.sh (bit-exact: same float code, same order);
  * torch's float64 CPU implementations through the committed golden
    fixtures (tests/golden/, written by make_golden.py);
  * what the mathematics fixes: central finite differences of the double
    forward, invariants (sum_c dx = 0, constant rows, odd-part identity of
    GELU), brute-force float64 sums;
and a planted-mistake test shows the checks reject a plausible error.
"""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
REF = O.ref()
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference absent)")


def rng(seed=0):
    return np.random.default_rng(seed)


# ----------------------------------------------------------------------------
# Against the reference's own CPU routines (oracle/_ref)
# ----------------------------------------------------------------------------

@needs_ref
def test_ln_forward_matches_reference_cpu_srand42():
    # FC/tests/test_layernorm.cu:29-39: rows=2048, cols=128, srand(42),
    # x = rand()/RAND_MAX - 0.5, gamma = 1, beta = 0, eps = 1e-5.
    rows, cols = 2048, 128
    (x,) = O.rand_unit_sequence(42, [rows * cols])
    x = x.reshape(rows, cols)
    gamma = np.ones(cols, np.float32)
    beta = np.zeros(cols, np.float32)
    y, m, s = O.layernorm_forward(x, gamma, beta, 1e-5)
    yr = np.empty_like(x)
    REF.ref_layernorm_cpu(O._p(x), O._p(gamma), O._p(beta), O._p(yr), rows, cols, 1e-5)
    assert np.array_equal(y.view(np.uint32), yr.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("rows,cols", [(64, 768), (7, 1600), (5, 33)])
def test_ln_forward_matches_reference_cpu_random(rows, cols):
    r = rng(1)
    x = r.standard_normal((rows, cols)).astype(np.float32)
    gamma = (1 + 0.02 * r.standard_normal(cols)).astype(np.float32)
    beta = (0.02 * r.standard_normal(cols)).astype(np.float32)
    y, _, _ = O.layernorm_forward(x, gamma, beta)
    yr = np.empty_like(x)
    REF.ref_layernorm_cpu(O._p(x), O._p(gamma), O._p(beta), O._p(yr), rows, cols, 1e-5)
    assert np.array_equal(y.view(np.uint32), yr.view(np.uint32))


@needs_ref
def test_ln_forward_f64_matches_reference_double():
    r = rng(2)
    rows, cols = 16, 96
    x = r.standard_normal((rows, cols)).astype(np.float32)
    gamma = (1 + 0.02 * r.standard_normal(cols)).astype(np.float32)
    beta = (0.02 * r.standard_normal(cols)).astype(np.float32)
    y, _, _ = O.layernorm_forward_f64(x, gamma, beta)
    x64, g64, b64 = (np.ascontiguousarray(a, np.float64) for a in (x, gamma, beta))
    yr = np.empty_like(x64)
    REF.ref_layernorm_f64(O._p(x64), O._p(g64), O._p(b64), O._p(yr), rows, cols, 1e-5)
    assert np.array_equal(y, yr)


@needs_ref
def test_embedding_matches_reference_cpu_srand42():
    # NC/tests/test_embedding.cu:46-59,103-110,145-155: V=512, D=128, B=16,
    # T=32; srand(42); table, tokens, grad_out, pos_table drawn in that order.
    V, D, B, T = 512, 128, 16, 32
    BT = B * T
    O.lib().orc_srand(42)
    table = np.empty(V * D, np.float32)
    O.lib().orc_fill_rand_unit(O._p(table), table.size)
    tokens = np.empty(BT, np.int32)
    O.lib().orc_fill_rand_tokens(O._p(tokens), BT, V)
    g = np.empty(BT * D, np.float32)
    O.lib().orc_fill_rand_unit(O._p(g), g.size)
    pos = np.empty(T * D, np.float32)
    O.lib().orc_fill_rand_unit(O._p(pos), pos.size)
    table, g, pos = table.reshape(V, D), g.reshape(BT, D), pos.reshape(T, D)

    out = O.embedding_forward(table, tokens)
    outr = np.empty_like(out)
    REF.ref_embedding_forward_cpu(O._p(table), O._p(tokens), O._p(outr), BT, D)
    assert np.array_equal(out.view(np.uint32), outr.view(np.uint32))

    gt = O.embedding_backward(g, tokens, np.zeros((V, D), np.float32))
    gtr = np.empty((V, D), np.float32)
    REF.ref_embedding_backward_cpu(O._p(g), O._p(tokens), O._p(gtr), BT, D, V)
    assert np.array_equal(gt.view(np.uint32), gtr.view(np.uint32))

    emb = O.pos_embedding_forward(pos, out, B, T)
    embr = outr.copy()
    REF.ref_pos_embedding_cpu(O._p(pos), O._p(embr), B, T, D)
    assert np.array_equal(emb.view(np.uint32), embr.view(np.uint32))


@needs_ref
def test_fill_pattern_matches_reference():
    for n, scale, shift in [(2048 * 128, 0.1, 0.0), (128, 0.03, 1.0), (512, 0.001, 0.0)]:
        a = O.fill_pattern(n, scale, shift)
        b = np.empty(n, np.float32)
        REF.ref_fill_pattern(O._p(b), n, scale, shift)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ----------------------------------------------------------------------------
# LayerNorm: golden fixtures (torch float64), invariants, finite differences
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("tag", ["c768", "c33"])
def test_ln_against_torch_golden(tag):
    d = np.load(os.path.join(GOLDEN, "layernorm_f64.npz"))
    x, gamma, beta, g = (d[f"{tag}_{k}"] for k in ("x", "gamma", "beta", "g"))
    y64, m64, s64 = O.layernorm_forward_f64(x, gamma, beta)
    np.testing.assert_allclose(y64, d[f"{tag}_y"], rtol=1e-12, atol=1e-12)
    dx64, dg64, db64 = O.layernorm_backward_f64(g, x, gamma)
    np.testing.assert_allclose(dx64, d[f"{tag}_dx"], rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(dg64, d[f"{tag}_dgamma"], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(db64, d[f"{tag}_dbeta"], rtol=1e-12, atol=1e-12)
    # float oracle against the same golden values (looser: float rounding)
    y, m, s = O.layernorm_forward(x, gamma, beta)
    np.testing.assert_allclose(y, d[f"{tag}_y"], rtol=1e-5, atol=2e-6)
    dx, dg, db = O.layernorm_backward(g, x, m, s, gamma)
    np.testing.assert_allclose(dx, d[f"{tag}_dx"], rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(dg, d[f"{tag}_dgamma"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(db, d[f"{tag}_dbeta"], rtol=1e-5, atol=1e-5)


def test_ln_constant_row_gives_beta_exactly():
    cols = 768
    x = np.full((3, cols), 0.75, np.float32)
    gamma = (1 + 0.02 * rng(3).standard_normal(cols)).astype(np.float32)
    beta = (0.02 * rng(4).standard_normal(cols)).astype(np.float32)
    y, m, s = O.layernorm_forward(x, gamma, beta)
    assert np.array_equal(y, np.broadcast_to(beta, y.shape))
    assert np.all(m == np.float32(0.75))
    assert np.allclose(s, 1 / np.sqrt(1e-5), rtol=1e-6)


def test_ln_unit_affine_moments():
    r = rng(5)
    rows, cols = 32, 768
    x = (3 * r.standard_normal((rows, cols)) + 2).astype(np.float32)
    y, m, s = O.layernorm_forward(x, np.ones(cols, np.float32), np.zeros(cols, np.float32))
    y64 = y.astype(np.float64)
    var = x.astype(np.float64).var(axis=1)
    assert np.all(np.abs(y64.mean(axis=1)) < 1e-6)
    np.testing.assert_allclose(y64.var(axis=1), var / (var + 1e-5), rtol=1e-5)
    np.testing.assert_allclose(m, x.astype(np.float64).mean(axis=1), rtol=1e-5, atol=1e-6)


def test_ln_backward_invariants_and_brute_force_columns():
    r = rng(6)
    rows, cols = 24, 257
    x = r.standard_normal((rows, cols)).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols)).astype(np.float32)
    dx, dg, db = O.layernorm_backward_f64(g, x, gamma)
    # sum_c dx = 0 for every row (the mean direction is projected out)
    assert np.all(np.abs(dx.sum(axis=1)) < 1e-10 * np.abs(dx).sum(axis=1).max())
    # brute-force column sums in float64
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=1, keepdims=True)
    rs = 1 / np.sqrt(((x64 - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    xh = (x64 - mu) * rs
    np.testing.assert_allclose(dg, (g * xh).sum(axis=0), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, g.astype(np.float64).sum(axis=0), rtol=1e-12, atol=1e-12)


def _ln_f64_np(x, gamma, beta, eps=1e-5):
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * gamma + beta


def test_ln_backward_finite_differences():
    # d/dx of sum(g * LN(x)) by central differences of the double forward
    r = rng(7)
    rows, cols = 3, 40
    x = r.standard_normal((rows, cols)).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32)
    beta = (0.1 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols)).astype(np.float32)
    dx, dg, db = O.layernorm_backward_f64(g, x, gamma)
    x64, g64, ga64, be64 = (a.astype(np.float64) for a in (x, g, gamma, beta))
    h = 1e-6
    num = np.zeros_like(x64)
    for i in range(rows):
        for j in range(cols):
            xp, xm = x64.copy(), x64.copy()
            xp[i, j] += h
            xm[i, j] -= h
            num[i, j] = ((g64 * _ln_f64_np(xp, ga64, be64)).sum()
                         - (g64 * _ln_f64_np(xm, ga64, be64)).sum()) / (2 * h)
    np.testing.assert_allclose(dx, num, rtol=1e-6, atol=1e-7)
    num_g = np.zeros(cols)
    for j in range(cols):
        gp, gm = ga64.copy(), ga64.copy()
        gp[j] += h
        gm[j] -= h
        num_g[j] = ((g64 * _ln_f64_np(x64, gp, be64)).sum()
                    - (g64 * _ln_f64_np(x64, gm, be64)).sum()) / (2 * h)
    np.testing.assert_allclose(dg, num_g, rtol=1e-6, atol=1e-7)


def test_ln_backward_float_oracle_close_to_f64_and_residual_mode():
    r = rng(8)
    rows, cols = 64, 768
    x = r.standard_normal((rows, cols)).astype(np.float32)
    gamma = (1 + 0.02 * r.standard_normal(cols)).astype(np.float32)
    beta = (0.02 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols)).astype(np.float32)
    _, m, s = O.layernorm_forward(x, gamma, beta)
    dx, dg, db = O.layernorm_backward(g, x, m, s, gamma)
    dx64, dg64, db64 = O.layernorm_backward_f64(g, x, gamma)
    np.testing.assert_allclose(dx, dx64, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dg, dg64, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(db, db64, rtol=1e-4, atol=1e-4)
    # residual mode adds dx onto grad_residual; dgamma/dbeta accumulate
    res0 = r.standard_normal((rows, cols)).astype(np.float32)
    dg0 = r.standard_normal(cols).astype(np.float32)
    rx, rdg, rdb = O.layernorm_backward(g, x, m, s, gamma, grad_x=res0, dgamma=dg0,
                                        dbeta=dg0, add_to_grad=True)
    assert np.array_equal(rx, res0 + dx)
    assert np.array_equal(rdg, dg0 + dg)


def test_residual_layernorm_is_add_then_layernorm():
    # FC/tests/test_fusion_benchmark.cu:162-165 pins the fused op as
    # residual_add followed by layernorm_forward_save.
    n = 2048 * 128
    a = O.fill_pattern(n, 0.1).reshape(2048, 128)
    b = O.fill_pattern(n, 0.08).reshape(2048, 128)
    gamma = O.fill_pattern(128, 0.03, 1.0)
    beta = O.fill_pattern(128, 0.02)
    r, y, m, s = O.residual_layernorm_forward(a, b, gamma, beta)
    assert np.array_equal(r, a + b)
    y2, m2, s2 = O.layernorm_forward(a + b, gamma, beta)
    assert np.array_equal(y, y2) and np.array_equal(m, m2) and np.array_equal(s, s2)


# ----------------------------------------------------------------------------
# GELU: golden fixture (torch float64), identities, finite differences
# ----------------------------------------------------------------------------

def test_gelu_against_torch_golden():
    d = np.load(os.path.join(GOLDEN, "gelu_tanh_f64.npz"))
    u, g = d["u"], d["g"]
    x = u.reshape(1, -1)
    zero_bias = np.zeros(u.size, np.float32)
    y64 = O.bias_gelu_forward_f64(x, zero_bias)[0]
    # torch evaluates 1 + tanh(z), which cancels in double below u = -7; the
    # oracle's logistic form does not, and the two agree to 1e-15 absolute
    # there (the golden values are the inexact ones).
    np.testing.assert_allclose(y64, d["y"], rtol=1e-13, atol=1e-15)
    gin64, _ = O.gelu_backward_with_bias_backward_f64(x, zero_bias, g.reshape(1, -1))
    np.testing.assert_allclose(gin64[0], d["gin"], rtol=1e-12, atol=1e-14)
    # float oracle (textbook float formula with tanhf)
    y = O.bias_gelu_forward(x, zero_bias)[0]
    np.testing.assert_allclose(y, d["y"], rtol=1e-5, atol=1e-6)
    gin, _ = O.gelu_backward_with_bias_backward(x, zero_bias, g.reshape(1, -1))
    np.testing.assert_allclose(gin[0], d["gin"], rtol=1e-4, atol=1e-6)


def test_gelu_identities():
    u = np.linspace(-8, 8, 1601).astype(np.float32)
    x = u.reshape(1, -1)
    zb = np.zeros(u.size, np.float32)
    y = O.bias_gelu_forward_f64(x, zb)[0]
    ym = O.bias_gelu_forward_f64(-x, zb)[0]
    # odd part: gelu(u) - gelu(-u) = u (exactly, since tanh is odd)
    np.testing.assert_allclose(y - ym, u.astype(np.float64), rtol=0, atol=1e-12)
    assert O.bias_gelu_forward_f64(np.zeros((1, 1), np.float32), np.zeros(1, np.float32))[0, 0] == 0
    d0, _ = O.gelu_backward_with_bias_backward_f64(np.zeros((1, 1), np.float32),
                                                   np.zeros(1, np.float32),
                                                   np.ones((1, 1), np.float32))
    assert d0[0, 0] == 0.5
    big = np.array([[30.0, -30.0]], np.float32)
    yb = O.bias_gelu_forward_f64(big, np.zeros(2, np.float32))[0]
    assert yb[0] == 30.0 and abs(yb[1]) < 1e-300


def test_gelu_backward_finite_differences_and_bias():
    r = rng(9)
    rows, cols = 6, 50
    x = (1.5 * r.standard_normal((rows, cols))).astype(np.float32)
    b = (0.02 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols)).astype(np.float32)
    gin, db = O.gelu_backward_with_bias_backward_f64(x, b, g)
    u = (x + b).astype(np.float64)
    h = 1e-6
    k0 = np.sqrt(2 / np.pi)

    def gelu(v):
        return 0.5 * v * (1 + np.tanh(k0 * (v + 0.044715 * v ** 3)))

    num = g * (gelu(u + h) - gelu(u - h)) / (2 * h)
    np.testing.assert_allclose(gin, num, rtol=1e-7, atol=1e-9)
    np.testing.assert_allclose(db, num.sum(axis=0), rtol=1e-7, atol=1e-9)
    ginf, dbf = O.gelu_backward_with_bias_backward(x, b, g)
    np.testing.assert_allclose(ginf, gin, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(dbf, db, rtol=1e-4, atol=1e-5)


# ----------------------------------------------------------------------------
# residual / bias / ReLU / embedding position backward: brute force
# ----------------------------------------------------------------------------

def test_elementwise_ops_against_numpy():
    r = rng(10)
    rows, cols = 37, 96
    a = r.standard_normal((rows, cols)).astype(np.float32)
    b = r.standard_normal((rows, cols)).astype(np.float32)
    bias = r.standard_normal(cols).astype(np.float32)
    assert np.array_equal(O.residual_add(a, b), a + b)
    assert np.array_equal(O.residual_add_with_bias(a, b, bias), (a + b) + bias)
    assert np.array_equal(O.bias_add(a, bias), a + bias)
    assert np.array_equal(O.relu_forward(a), np.where(a > 0, a, np.float32(0)))
    assert np.array_equal(O.relu_backward(a, b), np.where(a > 0, b, np.float32(0)))
    assert np.array_equal(O.bias_relu_forward(a, bias),
                          np.where(a + bias > 0, a + bias, np.float32(0)))
    gin, db = O.relu_backward_with_bias_backward(a, b)
    assert np.array_equal(gin, np.where(a > 0, b, np.float32(0)))
    np.testing.assert_allclose(db, gin.astype(np.float64).sum(axis=0), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(O.bias_backward(b), b.astype(np.float64).sum(axis=0), rtol=1e-5,
                               atol=1e-5)


def test_pos_embedding_backward_is_sum_over_batch():
    r = rng(11)
    B, T, D = 5, 7, 12
    g = r.standard_normal((B * T, D)).astype(np.float32)
    gp0 = r.standard_normal((T, D)).astype(np.float32)
    gp = O.pos_embedding_backward(g, gp0, B, T)
    expect = gp0.copy()
    for bb in range(B):
        expect = expect + g[bb * T:(bb + 1) * T]
    assert np.array_equal(gp, expect)


def test_embedding_backward_accumulates_in_token_order():
    r = rng(12)
    V, D, BT = 9, 16, 40
    tokens = r.integers(0, V, BT).astype(np.int32)
    g = r.standard_normal((BT, D)).astype(np.float32)
    gt0 = r.standard_normal((V, D)).astype(np.float32)
    gt = O.embedding_backward(g, tokens, gt0)
    expect = gt0.copy()
    for i in range(BT):
        expect[tokens[i]] = expect[tokens[i]] + g[i]
    assert np.array_equal(gt, expect)


# ----------------------------------------------------------------------------
# The checks above reject a plausible mistake (planted in a CPU copy).
# ----------------------------------------------------------------------------

def test_planted_mistake_in_ln_backward_is_caught():
    d = np.load(os.path.join(GOLDEN, "layernorm_f64.npz"))
    x, gamma, g = d["c768_x"].astype(np.float64), d["c768_gamma"].astype(np.float64), \
        d["c768_g"].astype(np.float64)
    mu = x.mean(axis=1, keepdims=True)
    rs = 1 / np.sqrt(((x - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    xh = (x - mu) * rs
    dh = g * gamma
    # dropped x_hat * mean(dh * x_hat) term
    wrong = rs * (dh - dh.mean(axis=1, keepdims=True))
    assert not np.allclose(wrong, d["c768_dx"], rtol=1e-4, atol=1e-5)
    # wrong sign of the projection term
    wrong2 = rs * (dh - dh.mean(axis=1, keepdims=True) + xh * (dh * xh).mean(axis=1, keepdims=True))
    assert not np.allclose(wrong2, d["c768_dx"], rtol=1e-4, atol=1e-5)
    right = rs * (dh - dh.mean(axis=1, keepdims=True) - xh * (dh * xh).mean(axis=1, keepdims=True))
    np.testing.assert_allclose(right, d["c768_dx"], rtol=1e-9, atol=1e-9)


def test_planted_mistake_in_gelu_derivative_is_caught():
    d = np.load(os.path.join(GOLDEN, "gelu_tanh_f64.npz"))
    u = d["u"].astype(np.float64)
    k0 = np.sqrt(2 / np.pi)
    t = np.tanh(k0 * (u + 0.044715 * u ** 3))
    # missing the factor 3 in the cubic term's derivative
    wrong = 0.5 * (1 + t) + 0.5 * u * (1 - t * t) * k0 * (1 + 0.044715 * u * u)
    assert not np.allclose(d["g"] * wrong, d["gin"], rtol=1e-4, atol=1e-6)


def test_embedding_backwards_are_adjoints_of_the_forwards():
    # <fwd(p), g> = <p, bwd(g)> for the linear maps p -> embedding_forward(p)
    # and p -> pos_embedding_forward(p, 0); the forwards are pinned bit-exact
    # against the reference's CPU routines above, so this pins the backwards
    # independently of their own loops.
    r = rng(13)
    V, D, B, T = 50, 24, 3, 7
    tokens = r.integers(0, V, B * T).astype(np.int32)
    table = r.standard_normal((V, D)).astype(np.float32)
    pos = r.standard_normal((T, D)).astype(np.float32)
    g = r.standard_normal((B * T, D)).astype(np.float32)
    lhs = float((O.embedding_forward(table, tokens).astype(np.float64) * g).sum())
    rhs = float((table.astype(np.float64)
                 * O.embedding_backward(g, tokens, np.zeros((V, D), np.float32))).sum())
    assert abs(lhs - rhs) <= 1e-4 * (abs(lhs) + 1)
    zeros = np.zeros((B * T, D), np.float32)
    lhs = float((O.pos_embedding_forward(pos, zeros, B, T).astype(np.float64) * g).sum())
    rhs = float((pos.astype(np.float64)
                 * O.pos_embedding_backward(g, np.zeros((T, D), np.float32), B, T)).sum())
    assert abs(lhs - rhs) <= 1e-4 * (abs(lhs) + 1)


# ----------------------------------------------------------------------------
# Softmax and cross-entropy
# ----------------------------------------------------------------------------

def _srand42_logits(rows, cols, with_targets):
    O.lib().orc_srand(42)
    x = np.empty(rows * cols, np.float32)
    O.lib().orc_fill_rand_unit(O._p(x), x.size)
    t = None
    if with_targets:
        t = np.empty(rows, np.int32)
        O.lib().orc_fill_rand_tokens(O._p(t), rows, cols)
    return x.reshape(rows, cols), t


@needs_ref
def test_softmax_and_cross_entropy_match_reference_cpu_srand42():
    # NC/tests/test_softmax_ce.cu:77-97 (softmax 256x512) and :125-141
    # (cross-entropy 128x4096), same srand(42) inputs
    x, _ = _srand42_logits(256, 512, False)
    ref = np.empty_like(x)
    REF.ref_softmax_cpu(O._p(x), O._p(ref), 256, 512)
    assert np.array_equal(O.softmax_forward(x).view(np.uint32), ref.view(np.uint32))

    logits, t = _srand42_logits(128, 4096, True)
    gref = np.empty_like(logits)
    lref = REF.ref_cross_entropy_cpu(O._p(logits), O._p(t), O._p(gref), 128, 4096)
    loss, grad = O.cross_entropy_cpu(logits, t)
    assert np.float32(loss).view(np.uint32) == np.float32(lref).view(np.uint32)
    assert np.array_equal(grad.view(np.uint32), gref.view(np.uint32))


@needs_ref
def test_softmax_matches_reference_cpu_random_shapes():
    r = rng(31)
    for rows, cols in ((3, 1), (5, 7), (4, 1025), (2, 50257)):
        x = (4 * r.standard_normal((rows, cols))).astype(np.float32)
        ref = np.empty_like(x)
        REF.ref_softmax_cpu(O._p(x), O._p(ref), rows, cols)
        assert np.array_equal(O.softmax_forward(x).view(np.uint32), ref.view(np.uint32))


def test_softmax_and_cross_entropy_against_torch_golden():
    d = np.load(os.path.join(GOLDEN, "softmax_ce_f64.npz"))
    logits, targets = d["logits"], d["targets"]
    np.testing.assert_allclose(O.softmax_forward_f64(logits), d["softmax"], rtol=1e-12,
                               atol=1e-300)
    l64, g64 = O.cross_entropy_f64(logits, targets)
    np.testing.assert_allclose(l64, d["loss"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(g64, d["grad"], rtol=1e-12, atol=1e-15)
    # the float routines at float accuracy
    np.testing.assert_allclose(O.softmax_forward(logits), d["softmax"], rtol=2e-6, atol=1e-9)
    losses, grad = O.cross_entropy_rows(logits, targets)
    # the reference kernel's loss is -log(p[t] + 1e-9), which departs from the
    # exact cross-entropy by about 1e-9 / p[t]: compare with that formula on
    # torch's float64 softmax, and bound the departure itself
    pt = d["softmax"][np.arange(len(targets)), targets]
    k64 = -np.log(pt + 1e-9)
    np.testing.assert_allclose(losses, k64, rtol=2e-6, atol=2e-6)
    assert (np.abs(k64 - d["loss"]) <= 1.01e-9 / pt).all()
    np.testing.assert_allclose(grad, d["grad"], rtol=2e-6, atol=2e-7)
    loss_cpu, grad_cpu = O.cross_entropy_cpu(logits, targets)
    assert abs(loss_cpu - d["loss"].mean()) <= 2e-6 * abs(d["loss"].mean())
    np.testing.assert_allclose(grad_cpu, d["grad"], rtol=2e-6, atol=2e-7)


def test_cross_entropy_rows_invariants():
    r = rng(33)
    logits = (2 * r.standard_normal((64, 777))).astype(np.float32)
    t = r.integers(0, 777, 64).astype(np.int32)
    losses, g = O.cross_entropy_rows(logits, t)
    assert (losses > 0).all()
    # rows of the gradient sum to zero (softmax sums to one)
    assert np.abs(g.astype(np.float64).sum(1)).max() < 5e-6
    # the gradient is the softmax minus the one-hot target
    onehot = np.zeros_like(g)
    onehot[np.arange(64), t] = 1
    np.testing.assert_allclose(g + onehot, O.softmax_forward(logits), rtol=1e-6, atol=1e-7)
    # scale is applied last, to every element
    _, gs = O.cross_entropy_rows(logits, t, 1 / 64)
    assert np.array_equal(gs.view(np.uint32), (g * np.float32(1 / 64)).view(np.uint32))
    # mean in row order
    acc = np.float32(0)
    for v in losses:
        acc = np.float32(acc + v)
    assert np.float32(O.loss_mean(losses)) == np.float32(acc / np.float32(64))
    # a target outside the row gives a NaN loss and no one-hot term
    bad = t.copy()
    bad[[3, 5]] = [-1, 777]
    lb, gb = O.cross_entropy_rows(logits, bad)
    assert np.isnan(lb[[3, 5]]).all() and np.array_equal(lb[:3], losses[:3])
    g0 = O.cross_entropy_rows(logits[3:4], np.array([0], np.int32))[1][0]
    np.testing.assert_array_equal(gb[3][1:], g0[1:])
    assert abs(gb[3][0] - (g0[0] + 1)) < 1e-7


def test_planted_mistake_in_cross_entropy_is_caught():
    d = np.load(os.path.join(GOLDEN, "softmax_ce_f64.npz"))
    logits, targets = d["logits"].astype(np.float64), d["targets"]
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    onehot = np.zeros_like(p)
    onehot[np.arange(p.shape[0]), targets] = 1
    # one-hot added instead of subtracted
    assert not np.allclose(p + onehot, d["grad"], rtol=1e-4, atol=1e-6)
    # loss taken at the wrong index (target - 1)
    wrong_loss = -np.log(p[np.arange(p.shape[0]), targets - 1])
    assert not np.allclose(wrong_loss, d["loss"], rtol=1e-4)
    np.testing.assert_allclose(p - onehot, d["grad"], rtol=1e-9, atol=1e-12)


# ----------------------------------------------------------------------------
# Optimizer step
# ----------------------------------------------------------------------------

def _torch_adam_f64(p, g_eff, m, v, lr, b1, b2, eps, steps_done):
    """torch.optim.Adam (float64, CPU): an independent implementation.  The
    moment buffers and step count are seeded from (m, v, steps_done)."""
    import torch
    pt = torch.tensor(p.astype(np.float64), requires_grad=True)
    opt = torch.optim.Adam([pt], lr=lr, betas=(b1, b2), eps=eps)
    pt.grad = torch.tensor(g_eff)
    if steps_done:
        st = opt.state[pt]
        st["step"] = torch.tensor(float(steps_done), dtype=torch.float64)
        st["exp_avg"] = torch.tensor(m.astype(np.float64))
        st["exp_avg_sq"] = torch.tensor(v.astype(np.float64))
    opt.step()
    st = opt.state[pt]
    return pt.detach().numpy(), st["exp_avg"].numpy(), st["exp_avg_sq"].numpy()


@pytest.mark.parametrize("step", [1, 7])
def test_adam_against_torch_optim_f64(step):
    r = rng(41 + step)
    n = 5000
    p = r.standard_normal(n).astype(np.float32)
    grad = (3 * r.standard_normal(n)).astype(np.float32)
    m = (0.1 * r.standard_normal(n)).astype(np.float32) if step > 1 else np.zeros(n, np.float32)
    v = (0.01 * r.random(n)).astype(np.float32) if step > 1 else np.zeros(n, np.float32)
    lr, b1, b2, eps, grad_scale = 3e-4, 0.9, 0.999, 1e-8, 0.5
    norm_sq = O.sumsq_f64(grad)
    max_norm = 1.0 / grad_scale
    clip = O.clip_scale(np.float32(norm_sq), max_norm)
    assert abs(clip - min(1.0, max_norm / np.sqrt(norm_sq))) < 1e-6
    bc1, bc2 = O.adam_bias_corrections(b1, b2, step)
    assert abs(bc1 - (1 - b1 ** step)) < 1e-6 and abs(bc2 - (1 - b2 ** step)) < 1e-6
    po, mo, vo = O.adam_clipped(p, grad, m, v, clip, lr, b1, b2, eps, bc1, bc2, grad_scale)
    g_eff = grad.astype(np.float64) * grad_scale * clip
    # torch gets the hyper-parameters as the float kernel sees them
    f = lambda a: float(np.float32(a))
    pt, mt, vt = _torch_adam_f64(p, g_eff, m, v, f(lr), f(b1), f(b2), f(eps), step - 1)
    np.testing.assert_allclose(mo, mt, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(vo, vt, rtol=1e-5, atol=1e-12)
    # the updated parameter: one float rounding of p - update (|p| ulp) plus
    # a relative error of the update (at most lr / (1 - b1^t) in size)
    bound = 1.2e-7 * np.abs(p) + 1e-4 * np.abs(pt - p) + 1e-12
    assert (np.abs(po - pt) <= bound).all()


def test_planted_mistake_in_adam_is_caught():
    r = rng(47)
    n = 2000
    p = r.standard_normal(n).astype(np.float32)
    grad = r.standard_normal(n).astype(np.float32)
    z = np.zeros(n, np.float32)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    f = lambda a: float(np.float32(a))
    pt, _, _ = _torch_adam_f64(p, grad.astype(np.float64), z, z, f(lr), f(b1), f(b2), f(eps), 0)
    # bias corrections left out (bc = 1)
    wrong, _, _ = O.adam_clipped(p, grad, z, z, 1.0, lr, b1, b2, eps, 1.0, 1.0, 1.0)
    bound = 1.2e-7 * np.abs(p) + 1e-4 * np.abs(pt - p) + 1e-12
    assert not (np.abs(wrong - pt) <= bound).all()
    bc1, bc2 = O.adam_bias_corrections(b1, b2, 1)
    right, _, _ = O.adam_clipped(p, grad, z, z, 1.0, lr, b1, b2, eps, bc1, bc2, 1.0)
    assert (np.abs(right - pt) <= bound).all()


def test_scale_and_sumsq():
    r = rng(49)
    x = r.standard_normal(1001).astype(np.float32)
    assert np.array_equal(O.scale_buffer(x, 0.25).view(np.uint32), (x * np.float32(0.25)).view(np.uint32))
    assert abs(O.sumsq_f64(x) - float((x.astype(np.float64) ** 2).sum())) < 1e-9


# ----------------------------------------------------------------------------
# 16-bit storage
# ----------------------------------------------------------------------------

def _f32_specials_and_random():
    bits = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0x7f800001,
                     0x33000000, 0x33000001, 0x33800000, 0x387fc000, 0x387fe000, 0x387ff000,
                     0x38800000, 0x477fe000, 0x477fefff, 0x477ff000, 0x477ff001, 0x7f7fffff,
                     0x3f800000, 0x3f801000, 0x3f802000, 0x3f803000, 0x3f808000, 0x00000001,
                     0x007fffff, 0x3effffff, 0xc0490fdb], np.uint32)
    r = rng(51)
    rand_bits = r.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    ranged = (r.standard_normal(100000) * np.exp(r.uniform(-30, 15, 100000))).astype(np.float32)
    return np.concatenate([bits.view(np.float32), rand_bits.view(np.float32), ranged])


def test_half_conversion_matches_numpy():
    # numpy's float32 -> float16 cast (round to nearest even) is independent
    x = _f32_specials_and_random()
    h = O.float_to_half(x)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(h[~nan], ref[~nan])
    assert np.isnan(O.half_to_float(h[nan])).all()
    # every half value converts back exactly
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = O.half_to_float(allh)
    fin = ~np.isnan(allh.view(np.float16))
    assert np.array_equal(f[fin].view(np.uint32), allh.view(np.float16)[fin].astype(np.float32).view(np.uint32))
    assert np.array_equal(O.float_to_half(f[fin]), allh[fin])


def test_bf16_conversion_matches_torch():
    import torch
    x = _f32_specials_and_random()
    b = O.float_to_bf16(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(b[~nan], ref[~nan])
    assert np.isnan(O.bf16_to_float(b[nan])).all()
    back = O.bf16_to_float(b[~nan])
    assert np.array_equal(back, torch.from_numpy(ref[~nan].view(np.int16).copy()).view(
        torch.bfloat16).float().numpy())


def test_fp16_storage_ops():
    r = rng(53)
    x = (2 * r.standard_normal((37, 129))).astype(np.float32)
    b = (0.1 * r.standard_normal(129)).astype(np.float32)
    h = O.bias_relu_forward_to_half(x, b)
    assert np.array_equal(h, np.maximum(x + b, np.float32(0)).astype(np.float16).view(np.uint16))
    g = r.standard_normal((37, 129)).astype(np.float32)
    gin, db = O.relu_backward_with_bias_backward_half_mask(h, g)
    gin2, db2 = O.relu_backward_with_bias_backward(O.half_to_float(h), g)
    assert np.array_equal(gin, gin2) and np.array_equal(db, db2)
