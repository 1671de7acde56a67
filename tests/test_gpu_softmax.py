"""GPU parity of softmax_forward and the softmax cross-entropy
(FINAL_CLEAN_CODE/src/kernels/activations.cu:394-532) against the CPU oracle:
  * softmax against NC/tests/test_softmax_ce.cu:26-44 restated
    (oracle.softmax_forward), forward tolerance, and float64;
  * cross-entropy against the reference kernel's arithmetic restated
    (oracle.cross_entropy_rows): per-row losses at the forward tolerance,
    gradients at the backward tolerance; the mean loss of
    cross_entropy_forward (host sum in row order) and of _v2 (device sum in
    a fixed order) at the forward tolerance;
  * the reference's own test cases (srand(42) inputs) with its own criteria;
  * row lengths across every register-resident shape and the long-row path,
    row counts that leave partial workgroups, invalid targets, large logits,
    determinism of repeated calls."""
import numpy as np
import pytest
import torch

import cme213_amd as M
import oracle as O
from gpu_util import dev_t, host, note
from tol import assert_bwd, assert_exact, assert_fwd, assert_fwd_within_oracle_error

pytestmark = pytest.mark.gpu


def _logits(rows, cols, seed, scale=3.0):
    r = np.random.default_rng(seed)
    x = (scale * r.standard_normal((rows, cols))).astype(np.float32)
    t = r.integers(0, cols, rows).astype(np.int32)
    return x, t


def test_reference_softmax_ce_test_cases(dev):
    # NC/tests/test_softmax_ce.cu:77-97 softmax 256x512, :125-141 CE 128x4096
    O.lib().orc_srand(42)
    x = np.empty(256 * 512, np.float32)
    O.lib().orc_fill_rand_unit(O._p(x), x.size)
    x = x.reshape(256, 512)
    X, Y = dev_t(x), torch.empty(256, 512, device="cuda")
    M.softmax_forward(X, Y, 256, 512)
    ref = O.softmax_forward(x)
    err = np.abs(host(Y) - ref).max()
    note(f"softmax 256x512 max err {err:.3e} (reference bound 1e-5)")
    assert err < 1e-5
    assert_fwd("softmax 256x512", host(Y), ref)

    O.lib().orc_srand(42)
    logits = np.empty(128 * 4096, np.float32)
    O.lib().orc_fill_rand_unit(O._p(logits), logits.size)
    t = np.empty(128, np.int32)
    O.lib().orc_fill_rand_tokens(O._p(t), 128, 4096)
    logits = logits.reshape(128, 4096)
    L, T, G = dev_t(logits), dev_t(t), torch.empty(128, 4096, device="cuda")
    loss = M.cross_entropy_forward(L, T, G, 128, 4096)
    loss_ref, grad_ref = O.cross_entropy_cpu(logits, t)
    grad_err = np.abs(host(G) - grad_ref).max()
    loss_err = abs(loss_ref - loss) / (abs(loss_ref) + 1e-8)
    note(f"cross_entropy 128x4096 loss {loss:.6f} vs {loss_ref:.6f} rel {loss_err:.3e}, "
         f"grad err {grad_err:.3e} (reference bounds 1e-2, 1e-4)")
    assert grad_err < 1e-4 and loss_err < 1e-2
    # and the kernel semantics at the library's tolerances
    lr, gr = O.cross_entropy_rows(logits, t)
    assert_bwd("ce grad 128x4096", host(G), gr)
    assert_fwd("ce mean loss", np.float32(loss), np.float32(O.loss_mean(lr)))


SM_SHAPES = [(1, 1), (7, 5), (33, 64), (5, 65), (9, 1000), (17, 1024), (3, 1025), (6, 2048),
             (10, 4096), (4, 5000), (3, 16384), (2, 16385), (3, 32768), (5, 50257), (2, 65536),
             (3, 70001)]


@pytest.mark.parametrize("rows,cols", SM_SHAPES)
def test_softmax_shapes(dev, rows, cols):
    note(f"softmax {rows}x{cols}")
    x, _ = _logits(rows, cols, rows * 7 + cols)
    X, Y = dev_t(x), torch.empty(rows, cols, device="cuda")
    M.softmax_forward(X, Y, rows, cols)
    y = host(Y)
    # long rows: the float oracle's sequential sum carries its own rounding
    # error (~sqrt(cols) ulp), which is added to the bound; the GPU is also
    # held to the plain tolerance against float64
    r64 = O.softmax_forward_f64(x)
    assert_fwd_within_oracle_error(f"softmax {rows}x{cols}", y, O.softmax_forward(x), r64)
    assert_fwd(f"softmax {rows}x{cols} vs f64", y, r64)


@pytest.mark.parametrize("rows,cols", SM_SHAPES)
def test_cross_entropy_shapes_v1_and_v2(dev, rows, cols):
    note(f"cross_entropy {rows}x{cols}")
    x, t = _logits(rows, cols, rows * 11 + cols)
    L, T = dev_t(x), dev_t(t)
    G1, G2 = torch.empty(rows, cols, device="cuda"), torch.empty(rows, cols, device="cuda")
    losses, lout = torch.empty(rows, device="cuda"), torch.empty(1, device="cuda")
    loss1 = M.cross_entropy_forward(L, T, G1, rows, cols)
    M.cross_entropy_forward_v2(L, T, G2, losses, lout, rows, cols)
    lr, gr = O.cross_entropy_rows(x, t)
    assert_bwd("grad (v1, scale 1)", host(G1), gr)
    _, gr2 = O.cross_entropy_rows(x, t, 1.0 / rows)
    assert_bwd("grad (v2, scale 1/batch)", host(G2), gr2)
    assert_fwd("per-row losses", host(losses), lr)
    mean_ref = np.float32(O.loss_mean(lr))
    assert_fwd("mean loss (v1, host)", np.float32(loss1), mean_ref)
    assert_fwd("mean loss (v2, device)", host(lout)[0], mean_ref)
    l64, g64 = O.cross_entropy_f64(x, t)
    assert_bwd("grad vs f64", host(G1), g64)
    # the kernel's loss is -log(p[t] + 1e-9): against float64, allow 1e-9 / p[t]
    pt = np.exp(-l64)
    assert (np.abs(host(losses) - l64) <= 1e-6 + 1e-5 * np.abs(l64) + 1.01e-9 / pt).all()


def test_cross_entropy_invalid_targets_large_logits_and_determinism(dev):
    rows, cols = 64, 3000
    x, t = _logits(rows, cols, 5, scale=30.0)   # large logits: needs the max shift
    x[4] += 1000.0
    t[[2, 9]] = [-1, cols]                      # invalid targets
    L, T = dev_t(x), dev_t(t)
    G, losses, lout = (torch.empty(rows, cols, device="cuda"), torch.empty(rows, device="cuda"),
                       torch.empty(1, device="cuda"))
    M.cross_entropy_forward_v2(L, T, G, losses, lout, rows, cols)
    lr, gr = O.cross_entropy_rows(x, t, 1.0 / rows)
    lg = host(losses)
    assert np.isnan(lg[[2, 9]]).all() and np.isnan(host(lout)[0])
    ok = np.ones(rows, bool)
    ok[[2, 9]] = False
    assert_fwd("losses (valid rows)", lg[ok], lr[ok])
    assert_bwd("grad incl. rows with invalid targets", host(G), gr)
    first = [host(G).copy(), lg.copy()]
    for _ in range(3):
        M.cross_entropy_forward_v2(L, T, G, losses, lout, rows, cols)
        assert_exact("repeat grad", host(G), first[0])
        assert_exact("repeat losses", host(losses), first[1])


def test_model_size_cross_entropy(dev):
    # B*T rows of GPT-2's 50257-way logits (a slice of the reference model's
    # loss: transformer.cu:402-407)
    rows, cols = 1024, 50257
    note(f"cross_entropy {rows}x{cols}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    L = torch.randn(rows, cols, device="cuda", generator=gen) * 2
    T = torch.randint(0, cols, (rows,), device="cuda", generator=gen, dtype=torch.int32)
    G, losses, lout = (torch.empty(rows, cols, device="cuda"), torch.empty(rows, device="cuda"),
                       torch.empty(1, device="cuda"))
    M.cross_entropy_forward_v2(L, T, G, losses, lout, rows, cols)
    x, t = host(L), host(T)
    O.set_threads(8)
    try:
        lr, gr = O.cross_entropy_rows(x, t, 1.0 / rows)
    finally:
        O.set_threads(1)
    assert_fwd("losses", host(losses), lr)
    assert_bwd("grad", host(G), gr)
    assert_fwd("mean loss", host(lout)[0], np.float32(O.loss_mean(lr)))
