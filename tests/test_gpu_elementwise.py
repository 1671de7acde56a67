"""GPU parity of the residual / bias / ReLU / GELU kernels against the CPU
oracle (restating FC/src/kernels/activations.cu:5-283 and the tanh-GELU
formula), through the C ABI.  Tolerances: tests/tol.py."""
import numpy as np
import pytest
import torch

import cme213_amd as M
import oracle as O
from gpu_util import dev_t, gelu_inputs, host, note
from tol import (assert_bwd, assert_bwd_within_oracle_error, assert_colsum, assert_exact,
                 assert_fwd, assert_fwd_within_oracle_error)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [8192 * 768, 4097, 1, 12])
def test_residual_add_bit_exact_and_in_place(dev, n):
    r = np.random.default_rng(n)
    a = r.standard_normal(n, dtype=np.float32)
    b = r.standard_normal(n, dtype=np.float32)
    ref = O.residual_add(a, b)
    A, B = dev_t(a), dev_t(b)
    out = torch.empty_like(A)
    M.residual_add(A, B, out, n)
    assert_exact("out", host(out), ref)
    M.residual_add(A, B, A, n)  # out aliases a, as FC/tests/test_fusion_benchmark.cu:234
    assert_exact("in-place", host(A), ref)


# (300, 16411): a prime width and more vectors than one walk step covers, so
# a column-fixed walk would need more than the maximum grid and the
# broadcast ops take the per-vector-column walk
@pytest.mark.parametrize("rows,cols", [(8192, 768), (4096, 1600), (17, 33), (3, 1),
                                       (70, 9001), (5, 40000), (300, 16411)])
def test_bias_and_relu_family(dev, rows, cols):
    note(f"bias/relu rows={rows} cols={cols}")
    r = np.random.default_rng(rows * 7 + cols)
    a = r.standard_normal((rows, cols), dtype=np.float32)
    x = r.standard_normal((rows, cols), dtype=np.float32)
    g = r.standard_normal((rows, cols), dtype=np.float32)
    bias = r.standard_normal(cols, dtype=np.float32)
    A, X, G, Bi = dev_t(a), dev_t(x), dev_t(g), dev_t(bias)

    out = torch.empty_like(A)
    M.residual_add_with_bias(A, X, Bi, out, rows, cols)
    assert_exact("residual_add_with_bias", host(out), O.residual_add_with_bias(a, x, bias))

    W = A.clone()
    M.bias_add(W, Bi, rows, cols)
    assert_exact("bias_add", host(W), O.bias_add(a, bias))

    M.bias_relu_forward(A, Bi, out, rows, cols)
    assert_exact("bias_relu_forward", host(out), O.bias_relu_forward(a, bias))

    M.relu_forward(A, out, rows * cols)
    assert_exact("relu_forward", host(out), O.relu_forward(a))

    M.relu_backward(A, G, out, rows * cols)
    assert_exact("relu_backward", host(out), O.relu_backward(a, g))

    db0 = r.standard_normal(cols, dtype=np.float32)
    gin_o, db_o = O.relu_backward_with_bias_backward(a, g, dbias=db0)
    DB = dev_t(db0)
    M.relu_backward_with_bias_backward(A, G, out, DB, rows, cols)
    assert_exact("relu_bwd grad_in", host(out), gin_o)
    assert_colsum("relu_bwd dbias", host(DB), db_o, gin_o)

    DB2 = dev_t(db0)
    M.bias_backward(G, DB2, rows, cols)
    assert_colsum("bias_backward", host(DB2), O.bias_backward(g, db0), g)


@pytest.mark.parametrize("rows,cols,seed", [
    (8192, 3072, 20261),
    (4096, 6400, 20264),   # config 4 GELU
    (8192, 768, 3),
    (37, 33, 4),
    (5, 1, 5),
    (1, 3072, 6),
    (300, 9001, 7),       # wider than the row-band kernels: column-slice path
    (700, 3000, 8),       # rows not a multiple of the band count
    (300, 16411, 9),      # prime width: the per-vector-column forward walk
])
def test_bias_gelu_forward_backward(dev, rows, cols, seed):
    # GELU has no reference implementation; its reference is the published
    # formula.  The parity target is the float64 evaluation of that formula
    # (orc_*_f64, pinned to torch's float64 GELU by the golden fixture), at the
    # stated fwd / bwd tolerances.  Against the float oracle (the textbook
    # float formula) the bound is the same tolerance plus that oracle's own
    # rounding error, which is large where 1 + tanhf(z) cancels (u < -4).
    note(f"gelu rows={rows} cols={cols} seed={seed}")
    x, b, g = gelu_inputs(rows, cols, seed)
    y64 = O.bias_gelu_forward_f64(x, b)
    gin64, db64 = O.gelu_backward_with_bias_backward_f64(x, b, g)
    y_o = O.bias_gelu_forward(x, b)
    db0 = np.full(cols, 0.125, np.float32)
    gin_o, db_o = O.gelu_backward_with_bias_backward(x, b, g, dbias=db0)

    X, Bi, G = dev_t(x), dev_t(b), dev_t(g)
    Y = torch.empty_like(X)
    M.bias_gelu_forward(X, Bi, Y, rows, cols)
    y = host(Y)
    assert_fwd("gelu y vs f64", y, y64)
    assert_fwd_within_oracle_error("gelu y vs float oracle", y, y_o, y64)
    GIN = torch.empty_like(X)
    DB = dev_t(db0)
    M.gelu_backward_with_bias_backward(X, Bi, G, GIN, DB, rows, cols)
    gin = host(GIN)
    assert_bwd("gelu grad_in vs f64", gin, gin64)
    assert_bwd_within_oracle_error("gelu grad_in vs float oracle", gin, gin_o, gin64)
    db = host(DB)
    assert_colsum("gelu dbias vs f64", db, db64 + db0.astype(np.float64), gin64,
                  approx_terms=True)
    assert_colsum("gelu dbias vs float oracle", db, db_o, gin64)

    e_gpu, e_orc = np.abs(y - y64).max(), np.abs(y_o - y64).max()
    eg_gpu, eg_orc = np.abs(gin - gin64).max(), np.abs(gin_o - gin64).max()
    note(f"  max err vs f64: fwd gpu {e_gpu:.3e} oracle {e_orc:.3e}; "
         f"bwd gpu {eg_gpu:.3e} oracle {eg_orc:.3e}")
    # the GPU form u*sigmoid(2z) is at least as accurate as the float formula
    assert e_gpu <= 2 * e_orc + 1e-7
    assert eg_gpu <= 2 * eg_orc + 1e-7


def test_gelu_special_values(dev):
    d = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                           "gelu_tanh_f64.npz"))
    u, g = d["u"], d["g"]
    n = u.size
    X = dev_t(u.reshape(1, n))
    Bz = torch.zeros(n, device=dev)
    Y = torch.empty_like(X)
    M.bias_gelu_forward(X, Bz, Y, 1, n)
    y = host(Y)[0]
    # golden (torch float64) values, fwd tolerance; plus exact limits
    assert_fwd("gelu golden", y, d["y"].astype(np.float32))
    assert y[0] == 0.0 and np.isfinite(y).all()
    big = u >= 20
    assert np.array_equal(y[big], u[big])
    GIN = torch.empty_like(X)
    DB = torch.zeros(n, device=dev)
    M.gelu_backward_with_bias_backward(X, Bz, dev_t(g.reshape(1, n)), GIN, DB, 1, n)
    gin = host(GIN)[0]
    assert np.isfinite(gin).all()
    assert_bwd("gelu grad golden", gin, d["gin"].astype(np.float32))
    # dbias = 0 + grad_in (a -0.0 gradient adds to +0.0)
    assert_exact("dbias of one row is grad_in", host(DB), gin + np.float32(0.0))


def test_gelu_extreme_values(dev):
    """Far tails and non-finite inputs: gelu(u) = 0 and gelu'(u) = 0 where
    |gelu| < 1e-36 (u <= -10.5, -inf), gelu(u) = u and gelu'(u) = 1 where
    the logistic factor is 1 in float (u >= 10.5, +inf), NaN stays NaN.
    (The clamped exponent once gave gelu(-1e38) = -1.2 and gelu'(1e20) =
    NaN.)"""
    u = np.array([-np.inf, -3e38, -1e38, -1e20, -1e14, -1e12, -1e4, -20.0, -10.5,
                  10.5, 20.0, 1e4, 1e12, 1e20, 1e38, 3e38, np.inf, np.nan], np.float32)
    n = u.size
    X = dev_t(u.reshape(1, n))
    Bz = torch.zeros(n, device=dev)
    Y = torch.empty_like(X)
    M.bias_gelu_forward(X, Bz, Y, 1, n)
    want_y = np.where(np.isnan(u), np.nan, np.where(u > 0, u, 0.0)).astype(np.float32)
    assert np.array_equal(host(Y)[0], want_y, equal_nan=True), host(Y)[0]
    GIN = torch.empty_like(X)
    DB = torch.zeros(n, device=dev)
    M.gelu_backward_with_bias_backward(X, Bz, torch.ones(1, n, device=dev), GIN, DB, 1, n)
    want_g = np.where(np.isnan(u), np.nan, np.where(u > 0, 1.0, 0.0)).astype(np.float32)
    assert np.array_equal(host(GIN)[0], want_g, equal_nan=True), host(GIN)[0]
    assert np.array_equal(host(DB), want_g, equal_nan=True)


def test_reduction_is_deterministic(dev):
    rows, cols = 8192, 3072
    x, b, g = gelu_inputs(rows, cols, 77)
    X, Bi, G = dev_t(x), dev_t(b), dev_t(g)
    res = []
    for _ in range(3):
        GIN = torch.empty_like(X)
        DB = torch.zeros(cols, device=dev)
        M.gelu_backward_with_bias_backward(X, Bi, G, GIN, DB, rows, cols)
        res.append((host(GIN), host(DB)))
    for r_ in res[1:]:
        assert_exact("grad_in repeat", r_[0], res[0][0])
        assert_exact("dbias repeat", r_[1], res[0][1])


def test_gelu_unaligned_scalar_path(dev):
    rows, cols = 64, 3072
    x, b, g = gelu_inputs(rows, cols, 88)
    X = torch.zeros(rows * cols + 1, device=dev)[1:].view(rows, cols)
    X.copy_(dev_t(x))
    Y = torch.zeros(rows * cols + 1, device=dev)[1:].view(rows, cols)
    M.bias_gelu_forward(X, dev_t(b), Y, rows, cols)
    assert_fwd("y", host(Y), O.bias_gelu_forward(x, b))
