"""GPU parity of a GPT-2 block's non-GEMM sequence chained over layers
(BASELINE configs 3 and 4), against the same chain run through the CPU
oracle.  Per layer: residual + LN1 (fused), residual + LN2 (fused), bias+GELU;
backward in reverse: GELU bwd + dbias, LN2 bwd accumulated into the
residual-stream gradient, LN1 bwd likewise (the call pattern of
FINAL_CLEAN_CODE/src/model/transformer.cu:360-364,534-538,573-577).  The
residual stream is carried from layer to layer, so errors would compound.

Full-size shapes run with few layers, full depth with fewer rows; the
column sums and the residual-stream gradient use the tolerances of tol.py."""
import numpy as np
import pytest
import torch

import oracle as O
from cme213_amd.workloads import BlockSequence
from gpu_util import host, note
from tol import assert_bwd, assert_colsum, assert_exact, assert_fwd

pytestmark = pytest.mark.gpu


def oracle_chain(r0, inp, params, gtop, L):
    """CPU oracle of BlockSequence.forward + backward."""
    acts = []
    r = r0
    for l in range(L):
        i, p = inp[l % len(inp)], params[l]
        r1, y1, m1, s1 = O.residual_layernorm_forward(r, i["a"], p["g1"], p["b1"])
        r2, y2, m2, s2 = O.residual_layernorm_forward(r1, i["m"], p["g2"], p["b2"])
        o64 = O.bias_gelu_forward_f64(i["h"], p["bias"])
        acts.append(dict(r1=r1, y1=y1, m1=m1, s1=s1, r2=r2, y2=y2, m2=m2, s2=s2, o64=o64))
        r = r2
    grads = [None] * L
    gres = gtop.copy()
    for l in reversed(range(L)):
        i, p, a = inp[l % len(inp)], params[l], acts[l]
        gin64, db64 = O.gelu_backward_with_bias_backward_f64(i["h"], p["bias"], i["gh"])
        gres, dg2, db2 = O.layernorm_backward(i["gy2"], a["r2"], a["m2"], a["s2"], p["g2"],
                                              grad_x=gres, add_to_grad=True)
        gres, dg1, db1 = O.layernorm_backward(i["gy1"], a["r1"], a["m1"], a["s1"], p["g1"],
                                              grad_x=gres, add_to_grad=True)
        grads[l] = dict(gin64=gin64, db64=db64, dg2=dg2, db2=db2, dg1=dg1, db1=db1)
    return r, acts, grads, gres


def _xhat_terms(g, x, m, s):
    xh = (x.astype(np.float64) - m[:, None].astype(np.float64)) * s[:, None]
    return g.astype(np.float64) * xh


@pytest.mark.parametrize("R,C,F,L,shared", [
    (8192, 768, 3072, 2, False),   # config 3 shapes, 2 layers
    (1024, 768, 3072, 12, True),   # config 3 depth
    (4096, 1600, 6400, 1, False),  # config 4 shapes, 1 layer
    (128, 1600, 6400, 48, True),   # config 4 depth
])
def test_block_sequence_chain(dev, R, C, F, L, shared):
    note(f"block chain R={R} C={C} F={F} layers={L}")
    bs = BlockSequence(R, C, F, L, seed=20263 + L, shared_inputs=shared)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    gtop = torch.randn(R, C, device="cuda", generator=gen)
    out = bs.forward()
    gres = bs.backward(gtop)
    torch.cuda.synchronize()

    inp = [{k: host(v) for k, v in d.items()} for d in bs.inp]
    params = [{k: host(v) for k, v in d.items()} for d in bs.params]
    r_o, acts_o, grads_o, gres_o = oracle_chain(host(bs.r0), inp, params, host(gtop), L)

    # forward: the residual stream is exact adds, so it matches bit for bit
    assert_exact("final residual stream", host(out), r_o)
    for l in range(L):
        a, ao = bs.act[l], acts_o[l]
        assert_exact(f"L{l} r1", host(a["r1"]), ao["r1"])
        assert_fwd(f"L{l} y1", host(a["y1"]), ao["y1"])
        assert_fwd(f"L{l} y2", host(a["y2"]), ao["y2"])
        assert_fwd(f"L{l} rstd2", host(a["s2"]), ao["s2"])
        assert_fwd(f"L{l} gelu", host(a["o"]), ao["o64"])
    # backward
    assert_bwd("residual-stream gradient", host(gres), gres_o)
    for l in range(L):
        i, a, ao, go, gr = inp[l % len(inp)], bs.act[l], acts_o[l], grads_o[l], bs.grads[l]
        assert_bwd(f"L{l} gelu grad_in", host(a["gin"]), go["gin64"])
        assert_colsum(f"L{l} dbias", host(gr["bias"]), go["db64"], go["gin64"])
        assert_colsum(f"L{l} dgamma2", host(gr["g2"]), go["dg2"],
                      _xhat_terms(i["gy2"], ao["r2"], ao["m2"], ao["s2"]))
        assert_colsum(f"L{l} dbeta2", host(gr["b2"]), go["db2"], i["gy2"])
        assert_colsum(f"L{l} dgamma1", host(gr["g1"]), go["dg1"],
                      _xhat_terms(i["gy1"], ao["r1"], ao["m1"], ao["s1"]))
        assert_colsum(f"L{l} dbeta1", host(gr["b1"]), go["db1"], i["gy1"])
