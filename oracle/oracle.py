"""numpy / ctypes front end of the CPU oracle (liboracle.so, built from oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product path (the HIP
library and its ctypes driver) never imports it.

Every function takes and returns numpy arrays (float32 / int32, C order,
copied if needed) and calls the C routine that restates the reference; see
oracle.c for the reference file:line each routine follows.  `ref()` returns
the library built from the reference's own CPU routines (oracle/_ref), or
None where it was not built.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_float, c_int, c_long, c_uint, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_cpu.so")

P = c_void_p
_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} not built (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        sigs = {
            "orc_set_threads": [c_int], "orc_get_threads": [],
            "orc_srand": [c_uint], "orc_fill_rand_unit": [P, c_long],
            "orc_fill_rand_tokens": [P, c_long, c_int],
            "orc_fill_pattern": [P, c_long, c_float, c_float],
            "orc_layernorm_forward": [P, P, P, P, P, P, c_int, c_int, c_float],
            "orc_layernorm_forward_f64": [P, P, P, P, P, P, c_int, c_int, c_double],
            "orc_residual_layernorm_forward": [P, P, P, P, P, P, P, P, c_int, c_int, c_float],
            "orc_layernorm_backward": [P, P, P, P, P, P, P, P, c_int, c_int, c_int],
            "orc_layernorm_backward_f64": [P, P, P, c_double, P, P, P, c_int, c_int],
            "orc_residual_add": [P, P, P, c_long],
            "orc_residual_add_with_bias": [P, P, P, P, c_int, c_int],
            "orc_bias_add": [P, P, c_int, c_int],
            "orc_relu_forward": [P, P, c_long],
            "orc_relu_backward": [P, P, P, c_long],
            "orc_bias_relu_forward": [P, P, P, c_int, c_int],
            "orc_bias_backward": [P, P, c_int, c_int],
            "orc_relu_backward_with_bias_backward": [P, P, P, P, c_int, c_int],
            "orc_bias_gelu_forward": [P, P, P, c_int, c_int],
            "orc_gelu_backward_with_bias_backward": [P, P, P, P, P, c_int, c_int],
            "orc_bias_gelu_forward_f64": [P, P, P, c_int, c_int],
            "orc_gelu_backward_with_bias_backward_f64": [P, P, P, P, P, c_int, c_int],
            "orc_embedding_forward": [P, P, P, c_int, c_int],
            "orc_embedding_backward": [P, P, P, c_int, c_int],
            "orc_pos_embedding_forward": [P, P, c_int, c_int, c_int],
            "orc_pos_embedding_backward": [P, P, c_int, c_int, c_int],
            "orc_softmax_forward": [P, P, c_int, c_int],
            "orc_softmax_forward_f64": [P, P, c_int, c_int],
            "orc_cross_entropy_cpu": [P, P, P, c_int, c_int],
            "orc_cross_entropy_rows": [P, P, P, P, c_int, c_int, c_float],
            "orc_loss_mean": [P, c_int],
            "orc_cross_entropy_f64": [P, P, P, P, c_int, c_int],
            "orc_scale_buffer": [P, c_float, c_long],
            "orc_sumsq_f64": [P, c_long],
            "orc_clip_scale": [c_float, c_float],
            "orc_adam_clipped": [P, P, P, P, c_float, c_float, c_float, c_float, c_float,
                                 c_float, c_float, c_float, c_long],
            "orc_adam_bias_corrections": [c_float, c_float, c_int, P, P],
            "orc_float_to_half": [P, P, c_long], "orc_half_to_float": [P, P, c_long],
            "orc_float_to_bf16": [P, P, c_long], "orc_bf16_to_float": [P, P, c_long],
            "orc_bias_relu_forward_to_half": [P, P, P, c_int, c_int],
            "orc_relu_backward_with_bias_backward_half_mask": [P, P, P, P, c_int, c_int],
        }
        restypes = {"orc_get_threads": c_int, "orc_cross_entropy_cpu": c_float,
                    "orc_loss_mean": c_float, "orc_sumsq_f64": c_double,
                    "orc_clip_scale": c_float}
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = restypes.get(name)
        _lib = L
    return _lib


def ref():
    """ctypes handle on oracle/_ref/libref_cpu.so (reference CPU routines) or None."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = ctypes.CDLL(REF_PATH)
        R.ref_layernorm_cpu.argtypes = [P, P, P, P, c_int, c_int, c_float]
        R.ref_layernorm_f64.argtypes = [P, P, P, P, c_int, c_int, c_double]
        R.ref_embedding_forward_cpu.argtypes = [P, P, P, c_int, c_int]
        R.ref_embedding_backward_cpu.argtypes = [P, P, P, c_int, c_int, c_int]
        R.ref_pos_embedding_cpu.argtypes = [P, P, c_int, c_int, c_int]
        R.ref_fill_pattern.argtypes = [P, c_int, c_float, c_float]
        R.ref_softmax_cpu.argtypes = [P, P, c_int, c_int]
        R.ref_cross_entropy_cpu.argtypes = [P, P, P, c_int, c_int]
        for fn in (R.ref_layernorm_cpu, R.ref_layernorm_f64, R.ref_embedding_forward_cpu,
                   R.ref_embedding_backward_cpu, R.ref_pos_embedding_cpu, R.ref_fill_pattern,
                   R.ref_softmax_cpu):
            fn.restype = None
        R.ref_cross_entropy_cpu.restype = c_float
        _ref = R
    return _ref


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a):
    return a.ctypes.data_as(c_void_p) if a is not None else None


def f32(a):
    return _c(a, np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


# ----- reference test-input generators ---------------------------------------

def rand_unit_sequence(seed: int, sizes):
    """srand(seed) then consecutive (float)rand()/RAND_MAX - 0.5f fills."""
    lib().orc_srand(seed)
    outs = []
    for n in sizes:
        v = np.empty(n, np.float32)
        lib().orc_fill_rand_unit(_p(v), n)
        outs.append(v)
    return outs


def fill_pattern(n: int, scale: float, shift: float = 0.0) -> np.ndarray:
    v = np.empty(n, np.float32)
    lib().orc_fill_pattern(_p(v), n, scale, shift)
    return v


# ----- LayerNorm ----------------------------------------------------------------

def layernorm_forward(x, gamma, beta, eps=1e-5):
    x, gamma, beta = f32(x), f32(gamma), f32(beta)
    rows, cols = x.shape
    y = np.empty_like(x)
    m = np.empty(rows, np.float32)
    s = np.empty(rows, np.float32)
    lib().orc_layernorm_forward(_p(x), _p(gamma), _p(beta), _p(y), _p(m), _p(s), rows, cols, eps)
    return y, m, s


def layernorm_forward_f64(x, gamma, beta, eps=1e-5):
    x, gamma, beta = f32(x), f32(gamma), f32(beta)
    rows, cols = x.shape
    y = np.empty(x.shape, np.float64)
    m = np.empty(rows, np.float64)
    s = np.empty(rows, np.float64)
    lib().orc_layernorm_forward_f64(_p(x), _p(gamma), _p(beta), _p(y), _p(m), _p(s), rows, cols,
                                    eps)
    return y, m, s


def residual_layernorm_forward(a, b, gamma, beta, eps=1e-5):
    a, b, gamma, beta = f32(a), f32(b), f32(gamma), f32(beta)
    rows, cols = a.shape
    r = np.empty_like(a)
    y = np.empty_like(a)
    m = np.empty(rows, np.float32)
    s = np.empty(rows, np.float32)
    lib().orc_residual_layernorm_forward(_p(a), _p(b), _p(gamma), _p(beta), _p(r), _p(y), _p(m),
                                         _p(s), rows, cols, eps)
    return r, y, m, s


def layernorm_backward(g, x, mean, inv_std, gamma, grad_x=None, dgamma=None, dbeta=None,
                       add_to_grad=False):
    """Returns (grad_x, dgamma, dbeta); the optional inputs are the initial
    values of the accumulated outputs (copied)."""
    g, x, mean, inv_std, gamma = f32(g), f32(x), f32(mean), f32(inv_std), f32(gamma)
    rows, cols = x.shape
    gx = f32(grad_x).copy() if grad_x is not None else np.zeros_like(x)
    dg = f32(dgamma).copy() if dgamma is not None else np.zeros(cols, np.float32)
    db = f32(dbeta).copy() if dbeta is not None else np.zeros(cols, np.float32)
    lib().orc_layernorm_backward(_p(g), _p(x), _p(mean), _p(inv_std), _p(gamma), _p(gx), _p(dg),
                                 _p(db), rows, cols, int(add_to_grad))
    return gx, dg, db


def layernorm_backward_f64(g, x, gamma, eps=1e-5):
    g, x, gamma = f32(g), f32(x), f32(gamma)
    rows, cols = x.shape
    gx = np.empty(x.shape, np.float64)
    dg = np.empty(cols, np.float64)
    db = np.empty(cols, np.float64)
    lib().orc_layernorm_backward_f64(_p(g), _p(x), _p(gamma), eps, _p(gx), _p(dg), _p(db), rows,
                                     cols)
    return gx, dg, db


# ----- residual / bias / activations -----------------------------------------

def residual_add(a, b):
    a, b = f32(a), f32(b)
    out = np.empty_like(a)
    lib().orc_residual_add(_p(a), _p(b), _p(out), a.size)
    return out


def residual_add_with_bias(residual, x, bias):
    residual, x, bias = f32(residual), f32(x), f32(bias)
    rows, cols = x.shape
    out = np.empty_like(x)
    lib().orc_residual_add_with_bias(_p(residual), _p(x), _p(bias), _p(out), rows, cols)
    return out


def bias_add(out, bias):
    out = f32(out).copy()
    bias = f32(bias)
    rows, cols = out.shape
    lib().orc_bias_add(_p(out), _p(bias), rows, cols)
    return out


def relu_forward(x):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_relu_forward(_p(x), _p(out), x.size)
    return out


def relu_backward(x, g):
    x, g = f32(x), f32(g)
    out = np.empty_like(x)
    lib().orc_relu_backward(_p(x), _p(g), _p(out), x.size)
    return out


def bias_relu_forward(x, bias):
    x, bias = f32(x), f32(bias)
    rows, cols = x.shape
    out = np.empty_like(x)
    lib().orc_bias_relu_forward(_p(x), _p(bias), _p(out), rows, cols)
    return out


def bias_backward(g, dbias=None):
    g = f32(g)
    rows, cols = g.shape
    db = f32(dbias).copy() if dbias is not None else np.zeros(cols, np.float32)
    lib().orc_bias_backward(_p(g), _p(db), rows, cols)
    return db


def relu_backward_with_bias_backward(mask, g, dbias=None):
    mask, g = f32(mask), f32(g)
    rows, cols = g.shape
    gin = np.empty_like(g)
    db = f32(dbias).copy() if dbias is not None else np.zeros(cols, np.float32)
    lib().orc_relu_backward_with_bias_backward(_p(mask), _p(g), _p(gin), _p(db), rows, cols)
    return gin, db


def bias_gelu_forward(x, bias):
    x, bias = f32(x), f32(bias)
    rows, cols = x.shape
    out = np.empty_like(x)
    lib().orc_bias_gelu_forward(_p(x), _p(bias), _p(out), rows, cols)
    return out


def gelu_backward_with_bias_backward(x, bias, g, dbias=None):
    x, bias, g = f32(x), f32(bias), f32(g)
    rows, cols = x.shape
    gin = np.empty_like(x)
    db = f32(dbias).copy() if dbias is not None else np.zeros(cols, np.float32)
    lib().orc_gelu_backward_with_bias_backward(_p(x), _p(bias), _p(g), _p(gin), _p(db), rows,
                                               cols)
    return gin, db


def bias_gelu_forward_f64(x, bias):
    x, bias = f32(x), f32(bias)
    rows, cols = x.shape
    out = np.empty(x.shape, np.float64)
    lib().orc_bias_gelu_forward_f64(_p(x), _p(bias), _p(out), rows, cols)
    return out


def gelu_backward_with_bias_backward_f64(x, bias, g):
    x, bias, g = f32(x), f32(bias), f32(g)
    rows, cols = x.shape
    gin = np.empty(x.shape, np.float64)
    db = np.empty(cols, np.float64)
    lib().orc_gelu_backward_with_bias_backward_f64(_p(x), _p(bias), _p(g), _p(gin), _p(db), rows,
                                                   cols)
    return gin, db


# ----- embedding -----------------------------------------------------------------

def embedding_forward(table, tokens):
    table = f32(table)
    tokens = _c(tokens, np.int32)
    bt = tokens.size
    dim = table.shape[1]
    out = np.empty((bt, dim), np.float32)
    lib().orc_embedding_forward(_p(table), _p(tokens), _p(out), bt, dim)
    return out


def embedding_backward(g, tokens, grad_table):
    g = f32(g)
    tokens = _c(tokens, np.int32)
    gt = f32(grad_table).copy()
    lib().orc_embedding_backward(_p(g), _p(tokens), _p(gt), tokens.size, gt.shape[1])
    return gt


def pos_embedding_forward(pos_table, emb, batch, seq):
    pos_table = f32(pos_table)
    emb = f32(emb).copy()
    lib().orc_pos_embedding_forward(_p(pos_table), _p(emb), batch, seq, pos_table.shape[1])
    return emb


def pos_embedding_backward(g, grad_pos, batch, seq):
    g = f32(g)
    gp = f32(grad_pos).copy()
    lib().orc_pos_embedding_backward(_p(g), _p(gp), batch, seq, gp.shape[1])
    return gp


# ----- softmax / cross-entropy -----------------------------------------------

def softmax_forward(x):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_softmax_forward(_p(x), _p(out), x.shape[0], x.shape[1])
    return out


def softmax_forward_f64(x):
    x = f32(x)
    out = np.empty(x.shape, np.float64)
    lib().orc_softmax_forward_f64(_p(x), _p(out), x.shape[0], x.shape[1])
    return out


def cross_entropy_cpu(logits, targets):
    """NC/tests/test_softmax_ce.cu:46-75: (mean loss, unscaled grad)."""
    logits = f32(logits)
    targets = _c(targets, np.int32)
    grad = np.empty_like(logits)
    loss = lib().orc_cross_entropy_cpu(_p(logits), _p(targets), _p(grad), logits.shape[0],
                                       logits.shape[1])
    return float(loss), grad


def cross_entropy_rows(logits, targets, scale=1.0):
    """The reference GPU kernel's arithmetic (activations.cu:438-477):
    (per-row losses, grad * scale)."""
    logits = f32(logits)
    targets = _c(targets, np.int32)
    grad = np.empty_like(logits)
    losses = np.empty(logits.shape[0], np.float32)
    lib().orc_cross_entropy_rows(_p(logits), _p(targets), _p(grad), _p(losses), logits.shape[0],
                                 logits.shape[1], scale)
    return losses, grad


def loss_mean(losses):
    losses = f32(losses)
    return float(lib().orc_loss_mean(_p(losses), losses.size))


def cross_entropy_f64(logits, targets):
    logits = f32(logits)
    targets = _c(targets, np.int32)
    grad = np.empty(logits.shape, np.float64)
    losses = np.empty(logits.shape[0], np.float64)
    lib().orc_cross_entropy_f64(_p(logits), _p(targets), _p(grad), _p(losses), logits.shape[0],
                                logits.shape[1])
    return losses, grad


# ----- optimizer step ----------------------------------------------------------

def scale_buffer(buf, scale):
    out = f32(buf).copy()
    lib().orc_scale_buffer(_p(out), scale, out.size)
    return out


def sumsq_f64(buf):
    buf = f32(buf)
    return float(lib().orc_sumsq_f64(_p(buf), buf.size))


def clip_scale(norm_sq, max_norm):
    return float(lib().orc_clip_scale(norm_sq, max_norm))


def adam_clipped(param, grad, m, v, clip, lr, beta1, beta2, eps, bc1, bc2, grad_scale):
    """Returns updated (param, m, v) copies."""
    p_, m_, v_ = f32(param).copy(), f32(m).copy(), f32(v).copy()
    grad = f32(grad)
    lib().orc_adam_clipped(_p(p_), _p(grad), _p(m_), _p(v_), clip, lr, beta1, beta2, eps, bc1,
                           bc2, grad_scale, p_.size)
    return p_, m_, v_


def adam_bias_corrections(beta1, beta2, step):
    b1, b2 = ctypes.c_float(0), ctypes.c_float(0)
    lib().orc_adam_bias_corrections(beta1, beta2, step, ctypes.byref(b1), ctypes.byref(b2))
    return b1.value, b2.value


# ----- 16-bit storage ----------------------------------------------------------

def float_to_half(x):
    x = f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_float_to_half(_p(x), _p(out), x.size)
    return out


def half_to_float(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_half_to_float(_p(h), _p(out), h.size)
    return out


def float_to_bf16(x):
    x = f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_float_to_bf16(_p(x), _p(out), x.size)
    return out


def bf16_to_float(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_float(_p(h), _p(out), h.size)
    return out


def bias_relu_forward_to_half(x, bias):
    x, bias = f32(x), f32(bias)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bias_relu_forward_to_half(_p(x), _p(bias), _p(out), x.shape[0], x.shape[1])
    return out


def relu_backward_with_bias_backward_half_mask(mask16, g, dbias=None):
    mask16, g = _c(mask16, np.uint16), f32(g)
    gin = np.empty_like(g)
    db = np.zeros(g.shape[1], np.float32) if dbias is None else f32(dbias).copy()
    lib().orc_relu_backward_with_bias_backward_half_mask(_p(mask16), _p(g), _p(gin), _p(db),
                                                         g.shape[0], g.shape[1])
    return gin, db
