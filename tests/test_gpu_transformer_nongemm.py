"""Caller integration: runs tests/cxx/transformer_nongemm, which issues the
non-GEMM calls of the reference's training step through include/kernels.h in
the order FINAL_CLEAN_CODE/src/model/transformer.cu:265-327 (forward) and
:475-584 (backward) issue them, with GEMM / attention outputs replaced by
fixed stand-in tensors.  The program also captures zero_grad + forward +
backward into a graph on the per-thread stream after three eager steps (as
main.cu:264-320 does) and requires every replay to match the eager step bit
for bit.

Here the eager step's outputs are compared with the same sequence run
through the CPU oracle: adds, gathers, ReLU and the embedding gradients
bit-exact; LN outputs and statistics at the forward tolerance; GELU against
the float64 formula; the residual-stream gradient at the backward tolerance;
column sums (db1, db2, dgamma, dbeta) at the column-sum tolerance.  The
"fp16" case is the reference's fp16-storage path (half copy of the FFN
activation, half-mask ReLU backward), with the half bits checked exactly."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from gpu_util import note
from tol import assert_bwd, assert_colsum, assert_exact, assert_fwd

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cxx", "transformer_nongemm")


def _load(d, name, shape, dtype=np.float32):
    return np.fromfile(os.path.join(d, name + ".bin"), dtype=dtype).reshape(shape)


@pytest.mark.parametrize("act", ["relu", "gelu", "fp16"])
def test_transformer_nongemm_sequence_and_graph_replay(dev, tmp_path, act):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built: run __graft_entry__.build() first")
    note(f"transformer_nongemm {act}")
    r = subprocess.run([EXE, str(tmp_path), act], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bit-identical to eager (3/3)" in r.stdout

    d = str(tmp_path)
    B, T, D, FF, V = (int(v) for v in np.fromfile(os.path.join(d, "shape.bin"), dtype=np.int32))
    BT = B * T
    ld = lambda n, *s: _load(d, n, s)
    tokens = _load(d, "tokens", (BT,), np.int32)
    tok_embed, pos_embed = ld("tok_embed", V, D), ld("pos_embed", T, D)
    ln1g, ln1b, ln2g, ln2b = ld("ln1_gamma", D), ld("ln1_beta", D), ld("ln2_gamma", D), ld("ln2_beta", D)
    b1, b2 = ld("b1", FF), ld("b2", D)
    s_attn, s_ffh, s_ffo = ld("s_attn_proj", BT, D), ld("s_ff_hidden", BT, FF), ld("s_ff_out", BT, D)
    s_gr2, s_gact = ld("s_grad_residual2", BT, D), ld("s_grad_ff_act", BT, FF)
    s_gl2, s_gl1 = ld("s_grad_ln2_out", BT, D), ld("s_grad_ln1_out", BT, D)

    # forward
    emb = O.pos_embedding_forward(pos_embed, O.embedding_forward(tok_embed, tokens), B, T)
    assert_exact("embedded", ld("embedded", BT, D), emb)
    y1, m1, s1 = O.layernorm_forward(emb, ln1g, ln1b)
    assert_fwd("ln1_out", ld("ln1_out", BT, D), y1)
    assert_fwd("ln1_mean", ld("ln1_mean", BT), m1)
    assert_fwd("ln1_inv_std", ld("ln1_inv_std", BT), s1)
    assert_exact("attn_proj (stand-in copy)", ld("attn_proj", BT, D), s_attn)
    r1, y2, m2, s2 = O.residual_layernorm_forward(emb, s_attn, ln2g, ln2b)
    assert_exact("residual1", ld("residual1", BT, D), r1)
    assert_fwd("ln2_out", ld("ln2_out", BT, D), y2)
    assert_fwd("ln2_inv_std", ld("ln2_inv_std", BT), s2)
    if act == "relu":
        act_ref = O.bias_relu_forward(s_ffh, b1)
        assert_exact("ff_act (bias+ReLU)", ld("ff_act", BT, FF), act_ref)
    elif act == "fp16":
        # CME213_FP16_STORAGE_ONLY: bias+ReLU in place, then the activation
        # round-trips through its half copy (transformer.cu:315-321)
        half_ref = O.float_to_half(O.bias_relu_forward(s_ffh, b1))
        assert_exact("ff_relu_half", _load(d, "ff_relu_half", (-1,), np.uint16)[:BT * FF],
                     half_ref.reshape(-1))
        assert_exact("ff_hidden (ReLU through half)", ld("ff_hidden", BT, FF),
                     O.half_to_float(half_ref))
    else:
        assert_fwd("ff_act (bias+GELU)", ld("ff_act", BT, FF), O.bias_gelu_forward_f64(s_ffh, b1))
    assert_exact("residual2", ld("residual2", BT, D), O.residual_add_with_bias(r1, s_ffo, b2))

    # backward; the flat gradient buffer holds dtok, dpos, dln1 g/b, dln2 g/b, db1, db2
    grads = ld("all_grads", V * D + T * D + 4 * D + FF + D)
    o = 0
    parts = {}
    for name, n in (("dtok", V * D), ("dpos", T * D), ("dln1_g", D), ("dln1_b", D),
                    ("dln2_g", D), ("dln2_b", D), ("db1", FF), ("db2", D)):
        parts[name] = grads[o:o + n]
        o += n
    assert_colsum("db2", parts["db2"], s_gr2.astype(np.float64).sum(0), s_gr2)
    if act == "relu":
        gin, _ = O.relu_backward_with_bias_backward(act_ref, s_gact)
        assert_exact("grad_ff_hidden (ReLU)", ld("grad_ff_hidden", BT, FF), gin)
        assert_colsum("db1", parts["db1"], gin.astype(np.float64).sum(0), gin)
    elif act == "fp16":
        gin, _ = O.relu_backward_with_bias_backward_half_mask(half_ref, s_gact)
        assert_exact("grad_ff_hidden (half mask)", ld("grad_ff_hidden", BT, FF), gin)
        assert_colsum("db1", parts["db1"], gin.astype(np.float64).sum(0), gin)
    else:
        gin64, db64 = O.gelu_backward_with_bias_backward_f64(s_ffh, b1, s_gact)
        assert_bwd("grad_ff_hidden (GELU)", ld("grad_ff_hidden", BT, FF), gin64)
        assert_colsum("db1", parts["db1"], db64, gin64, approx_terms=True)
    gres, dg2, db2ln = O.layernorm_backward(s_gl2, r1, m2, s2, ln2g, grad_x=s_gr2.copy(),
                                            add_to_grad=True)
    gres, dg1, db1ln = O.layernorm_backward(s_gl1, emb, m1, s1, ln1g, grad_x=gres,
                                            add_to_grad=True)
    gpu_gres = ld("grad_residual2", BT, D)
    assert_bwd("grad_residual2 after LN2 and LN1 backward", gpu_gres, gres)
    xh2 = (r1.astype(np.float64) - m2[:, None]) * s2[:, None]
    xh1 = (emb.astype(np.float64) - m1[:, None]) * s1[:, None]
    assert_colsum("dln2_gamma", parts["dln2_g"], dg2, s_gl2 * xh2)
    assert_colsum("dln2_beta", parts["dln2_b"], db2ln, s_gl2)
    assert_colsum("dln1_gamma", parts["dln1_g"], dg1, s_gl1 * xh1)
    assert_colsum("dln1_beta", parts["dln1_b"], db1ln, s_gl1)
    # the embedding gradients are bit-exact given the GPU's residual-stream gradient
    assert_exact("dtok_embed", parts["dtok"].reshape(V, D),
                 O.embedding_backward(gpu_gres, tokens, np.zeros((V, D), np.float32)))
    assert_exact("dpos_embed", parts["dpos"].reshape(T, D),
                 O.pos_embedding_backward(gpu_gres, np.zeros((T, D), np.float32), B, T))
