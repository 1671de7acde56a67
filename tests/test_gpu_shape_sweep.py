"""Seeded shape sweep: the layer kernels on shapes drawn at random (fixed
seed) across the dispatch boundaries of the library, against the CPU oracle
at the stated tolerances (tests/tol.py).

The boundaries crossed: rows-per-wave choice of the LN forward (6144 rows,
6M and 16M elements, 4096-wide rows), one / four / eight waves per LN
backward row (2048 and 8192 columns), the register-resident widths against
the block-per-row fallbacks, vector (W = 4) against scalar columns (width not
a multiple of 4, or a tensor that starts 4 bytes into its allocation), the
flat against the row-band form of the bias operators (one to four column
vectors per row-band thread), and the embedding
backward's owner count (a power of two from about 32 tokens each)."""
import numpy as np
import pytest
import torch

import cme213_amd as M
import oracle as O
from gpu_util import dev_t, host, note
from tol import assert_bwd, assert_colsum, assert_exact, assert_fwd

pytestmark = pytest.mark.gpu


def _shapes(seed, n, max_elems, fixed):
    """n (rows, cols, offset) triples: log-uniform rows and cols with
    rows * cols <= max_elems, plus the fixed boundary cases."""
    r = np.random.default_rng(seed)
    out = list(fixed)
    while len(out) < n + len(fixed):
        cols = int(np.exp(r.uniform(0, np.log(9000))))
        rows = int(np.exp(r.uniform(0, np.log(20000))))
        if rows * cols > max_elems or rows < 1 or cols < 1:
            continue
        out.append((rows, cols, int(r.integers(0, 2))))
    return out


def _on_device(a, offset):
    """Copy to the GPU; with offset 1 the tensor starts 4 bytes into its
    allocation, so the kernels take their unaligned (scalar) path."""
    flat = np.ascontiguousarray(a).reshape(-1)
    buf = torch.empty(flat.size + offset, dtype=torch.float32, device="cuda:0")
    view = buf[offset:]
    view.copy_(torch.from_numpy(flat))
    return view.view(a.shape)


LN_SHAPES = _shapes(101, 10, 6 << 20, [(6144, 1024, 0), (6143, 1024, 0), (8192, 4096, 0),
                                       (2050, 2052, 0), (3, 8192, 1), (2, 8196, 0)])


@pytest.mark.parametrize("rows,cols,offset", LN_SHAPES)
def test_layernorm_shape_sweep(dev, rows, cols, offset):
    note(f"LN sweep rows={rows} cols={cols} offset={offset}")
    r = np.random.default_rng(rows * 131 + cols)
    x = r.standard_normal((rows, cols), dtype=np.float32)
    gamma = (1 + 0.02 * r.standard_normal(cols)).astype(np.float32)
    beta = (0.02 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols), dtype=np.float32)
    res = r.standard_normal((rows, cols), dtype=np.float32)

    y_o, m_o, s_o = O.layernorm_forward(x, gamma, beta)
    X, G, B = _on_device(x, offset), dev_t(gamma), dev_t(beta)
    Y = _on_device(np.zeros_like(x), offset)
    Mn, Rs = torch.empty(rows, device=dev), torch.empty(rows, device=dev)
    M.layernorm_forward_save(X, G, B, Y, Mn, Rs, rows, cols, 1e-5)
    assert_fwd("y", host(Y), y_o)
    assert_fwd("rstd", host(Rs), s_o)

    # backward accumulating into an existing residual gradient
    dx_o, dg_o, db_o = O.layernorm_backward(g, x, m_o, s_o, gamma, grad_x=res.copy(),
                                            add_to_grad=True)
    GR = _on_device(res, offset)
    DG, DB = torch.zeros(cols, device=dev), torch.zeros(cols, device=dev)
    M.layernorm_backward_residual(_on_device(g, offset), X, dev_t(m_o), dev_t(s_o), G, GR, DG,
                                  DB, rows, cols)
    assert_bwd("grad_residual", host(GR), dx_o)
    xh = (x.astype(np.float64) - m_o[:, None]) * s_o[:, None]
    assert_colsum("dgamma", host(DG), dg_o, g.astype(np.float64) * xh)
    assert_colsum("dbeta", host(DB), db_o, g)


# The fixed cases include rows of 3 and 4 column vectors per row-band thread
# (12288 and 16000 columns) with more rows than row bands, where the kernel's
# workgroup and grid sizes (passed as arguments) set every thread's columns
# and rows.
GELU_SHAPES = _shapes(202, 10, 4 << 20, [(8192, 3, 0), (1, 16384, 0), (513, 4097, 1),
                                         (4096, 6400, 0), (350, 12288, 0), (300, 16000, 0)])


@pytest.mark.parametrize("rows,cols,offset", GELU_SHAPES)
def test_bias_gelu_and_relu_shape_sweep(dev, rows, cols, offset):
    note(f"GELU/ReLU sweep rows={rows} cols={cols} offset={offset}")
    r = np.random.default_rng(rows * 257 + cols)
    x = (1.5 * r.standard_normal((rows, cols), dtype=np.float32)).astype(np.float32)
    b = (0.02 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols), dtype=np.float32)
    X, Bi, Gd = _on_device(x, offset), dev_t(b), _on_device(g, offset)

    Y = _on_device(np.zeros_like(x), offset)
    M.bias_gelu_forward(X, Bi, Y, rows, cols)
    assert_fwd("gelu y", host(Y), O.bias_gelu_forward_f64(x, b))
    gin64, db64 = O.gelu_backward_with_bias_backward_f64(x, b, g)
    GIN = _on_device(np.zeros_like(x), offset)
    DBI = torch.zeros(cols, device=dev)
    M.gelu_backward_with_bias_backward(X, Bi, Gd, GIN, DBI, rows, cols)
    assert_bwd("gelu grad_in", host(GIN), gin64)
    assert_colsum("gelu dbias", host(DBI), db64, gin64, approx_terms=True)

    M.bias_relu_forward(X, Bi, Y, rows, cols)
    act = O.bias_relu_forward(x, b)
    assert_exact("bias_relu", host(Y), act)
    gin, _ = O.relu_backward_with_bias_backward(act, g)
    DBI.zero_()
    M.relu_backward_with_bias_backward(Y, Gd, GIN, DBI, rows, cols)
    assert_exact("relu grad_in", host(GIN), gin)
    assert_colsum("relu dbias", host(DBI), gin.astype(np.float64).sum(0), gin)


@pytest.mark.parametrize("seed", range(6))
def test_embedding_backward_shape_sweep(dev, seed):
    r = np.random.default_rng(300 + seed)
    V = int(np.exp(r.uniform(np.log(2), np.log(60000))))
    D = int(r.integers(1, 1100))
    n = int(np.exp(r.uniform(0, np.log(40000))))
    vocab_arg = V if seed % 2 == 0 else 0
    note(f"embedding sweep V={V} D={D} n={n} vocab_arg={vocab_arg}")
    ids = r.integers(0, V, n).astype(np.int32)
    g = r.standard_normal((n, D), dtype=np.float32)
    t0 = r.standard_normal((V, D), dtype=np.float32)
    T = dev_t(t0)
    M.embedding_backward(dev_t(g), dev_t(ids), T, n, D, vocab_arg)
    assert_exact("dwte", host(T), O.embedding_backward(g, ids, t0))
