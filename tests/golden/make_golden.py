"""Writes the golden fixtures under tests/golden/ from torch's CPU float64
implementations (a third-party library, independent of both the reference
and this repository's oracle):

  gelu_tanh_f64.npz   u, g -> gelu_tanh(u), g * gelu_tanh'(u)
                      (torch.nn.functional.gelu(approximate="tanh") + autograd)
  layernorm_f64.npz   x, gamma, beta, g -> y, dx, dgamma, dbeta for two shapes
                      (torch.nn.functional.layer_norm + autograd, eps=1e-5)
  softmax_ce_f64.npz  logits, targets -> softmax, per-row cross-entropy, and
                      its gradient (torch.softmax, torch.nn.functional
                      .cross_entropy(reduction="none") + autograd)

Inputs are float32 values (stored as float32) so the float paths can consume
them; torch computes in float64 on those exact values.  Re-run with
`python tests/golden/make_golden.py [name ...]` (deterministic; seeds fixed
below; with names, only those fixtures are rewritten).
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def gelu_fixture(rng):
    special = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-7, -1e-7, 0.5, -0.5, 1.0, -1.0, 2.0, -2.0,
                        3.0, -3.0, 5.0, -5.0, 8.0, -8.0, 10.0, -10.0, 12.0, -12.0, 20.0, -20.0,
                        50.0, -50.0], np.float32)
    grid = np.linspace(-12.0, 12.0, 961, dtype=np.float32)
    rnd = (rng.standard_normal(2000) * 1.5).astype(np.float32)
    u = np.concatenate([special, grid, rnd]).astype(np.float32)
    g = rng.standard_normal(u.size).astype(np.float32)
    ut = torch.tensor(u.astype(np.float64), requires_grad=True)
    y = torch.nn.functional.gelu(ut, approximate="tanh")
    y.backward(torch.tensor(g.astype(np.float64)))
    return dict(u=u, g=g, y=y.detach().numpy(), gin=ut.grad.numpy())


def ln_case(rng, rows, cols, tag):
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[0] = 0.25  # a constant row: y must equal beta
    gamma = (1.0 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    beta = (0.02 * rng.standard_normal(cols)).astype(np.float32)
    g = rng.standard_normal((rows, cols)).astype(np.float32)
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    gt = torch.tensor(gamma.astype(np.float64), requires_grad=True)
    bt = torch.tensor(beta.astype(np.float64), requires_grad=True)
    y = torch.nn.functional.layer_norm(xt, (cols,), gt, bt, eps=1e-5)
    y.backward(torch.tensor(g.astype(np.float64)))
    return {f"{tag}_x": x, f"{tag}_gamma": gamma, f"{tag}_beta": beta, f"{tag}_g": g,
            f"{tag}_y": y.detach().numpy(), f"{tag}_dx": xt.grad.numpy(),
            f"{tag}_dgamma": gt.grad.numpy(), f"{tag}_dbeta": bt.grad.numpy()}


def softmax_ce_fixture():
    rng = np.random.default_rng(20267)
    rows, cols = 12, 1000
    logits = (3.0 * rng.standard_normal((rows, cols))).astype(np.float32)
    logits[1] = 0.5            # a constant row: uniform softmax
    logits[2, 7] = 60.0        # a dominant logit
    logits[3] -= 80.0          # large negative offset (needs the max shift)
    targets = rng.integers(0, cols, rows).astype(np.int32)
    targets[2] = 7
    lt = torch.tensor(logits.astype(np.float64), requires_grad=True)
    sm = torch.softmax(lt, dim=1)
    loss = torch.nn.functional.cross_entropy(lt, torch.tensor(targets.astype(np.int64)),
                                             reduction="none")
    loss.sum().backward()
    return dict(logits=logits, targets=targets, softmax=sm.detach().numpy(),
                loss=loss.detach().numpy(), grad=lt.grad.numpy())


def main(names):
    if not names or "gelu_tanh_f64" in names or "layernorm_f64" in names:
        rng = np.random.default_rng(20260)
        np.savez_compressed(os.path.join(HERE, "gelu_tanh_f64.npz"), **gelu_fixture(rng))
        d = {}
        d.update(ln_case(rng, 16, 768, "c768"))
        d.update(ln_case(rng, 9, 33, "c33"))
        np.savez_compressed(os.path.join(HERE, "layernorm_f64.npz"), **d)
    if not names or "softmax_ce_f64" in names:
        np.savez_compressed(os.path.join(HERE, "softmax_ce_f64.npz"), **softmax_ce_fixture())
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    import sys
    main(sys.argv[1:])
