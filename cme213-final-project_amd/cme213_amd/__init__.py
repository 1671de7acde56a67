"""ctypes driver for libcme213_amd.so, the gfx950 fused non-GEMM layer kernels.

The Python functions mirror the reference's C++ kernel interface
(FINAL_CLEAN_CODE/include/kernels.h; cited per function in
include/mi_kernels.h): same names, same argument order and meaning, same
overwrite / accumulate (`+=`) contract.  Arguments that are device buffers
accept either a torch CUDA tensor (its data_ptr() is passed; it must be
contiguous and of the stated dtype) or a raw device address as int.  A
failure raises MIError carrying the library's status code and message; there
is no fallback path: if the shared library is missing the import fails.

Every call is asynchronous on `stream` (a raw hipStream_t as int); the
default is torch's current stream on the current device, so torch events and
synchronisation see the kernels.
"""
from __future__ import annotations

import ctypes
import os
import re
from ctypes import c_float, c_int, c_longlong, c_size_t, c_void_p, c_char_p

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
REPO_ROOT = os.path.dirname(PKG_ROOT)
LIB_PATH = os.path.join(PKG_ROOT, "libcme213_amd.so")
HEADERS = [os.path.join(REPO_ROOT, "include", "mi_kernels.h"),
           os.path.join(REPO_ROOT, "include", "kernels.h")]

MI_OK = 0
MI_ERR_INVALID_ARG = -1
MI_ERR_CAPTURE_ALLOC = -2


class MIError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
        "(the HIP library is required; there is no CPU fallback)")

# torch wheels bundle their own libamdhip64 / libhsa-runtime64 (same sonames
# as /opt/rocm's).  Loading torch first makes this library bind to the runtime
# torch already holds, so one process never initialises two HIP runtimes
# (which leaves one of them without devices).  Without torch, the system
# runtime is used.
try:
    import torch  # noqa: F401
except ImportError:
    pass

lib = ctypes.CDLL(LIB_PATH)

P = c_void_p
_SIGS = {
    # runtime
    "mi_last_error": (c_char_p, []),
    "mi_version": (c_char_p, []),
    "mi_device_count": (c_int, [P]),
    "mi_set_device": (c_int, [c_int]),
    "mi_malloc": (c_int, [P, c_size_t]),
    "mi_free": (c_int, [P]),
    "mi_memcpy_h2d": (c_int, [P, P, c_size_t]),
    "mi_memcpy_d2h": (c_int, [P, P, c_size_t]),
    "mi_memset_zero": (c_int, [P, c_size_t, P]),
    "mi_stream_sync": (c_int, [P]),
    "mi_device_sync": (c_int, []),
    "mi_workspace_reserve": (c_int, [c_size_t]),
    "mi_workspace_bytes": (c_size_t, []),
    "mi_workspace_reserve_stream": (c_int, [c_size_t, P]),
    "mi_workspace_bytes_stream": (c_size_t, [P]),
    "mi_workspace_release": (c_int, []),
    "mi_layernorm_backward_workspace": (c_size_t, [c_int, c_int]),
    "mi_bias_backward_workspace": (c_size_t, [c_int, c_int]),
    "mi_embedding_backward_workspace": (c_size_t, [c_int]),
    # LayerNorm
    "mi_layernorm_forward": (c_int, [P, P, P, P, c_int, c_int, c_float, P]),
    "mi_layernorm_forward_save": (c_int, [P, P, P, P, P, P, c_int, c_int, c_float, P]),
    "mi_residual_layernorm_forward_save":
        (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_float, P]),
    "mi_layernorm_backward": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, P]),
    "mi_layernorm_backward_residual": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, P]),
    "mi_layernorm_backward_noalloc": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, P]),
    # residual / bias / activations
    "mi_residual_add": (c_int, [P, P, P, c_longlong, P]),
    "mi_residual_add_with_bias": (c_int, [P, P, P, P, c_int, c_int, P]),
    "mi_bias_add": (c_int, [P, P, c_int, c_int, P]),
    "mi_relu_forward": (c_int, [P, P, c_longlong, P]),
    "mi_relu_backward": (c_int, [P, P, P, c_longlong, P]),
    "mi_bias_relu_forward": (c_int, [P, P, P, c_int, c_int, P]),
    "mi_relu_backward_with_bias_backward": (c_int, [P, P, P, P, c_int, c_int, P]),
    "mi_bias_backward": (c_int, [P, P, c_int, c_int, P]),
    "mi_bias_gelu_forward": (c_int, [P, P, P, c_int, c_int, P]),
    "mi_gelu_backward_with_bias_backward": (c_int, [P, P, P, P, P, c_int, c_int, P]),
    # embedding
    "mi_embedding_forward": (c_int, [P, P, P, c_int, c_int, c_int, P]),
    "mi_embedding_backward": (c_int, [P, P, P, c_int, c_int, c_int, P]),
    "mi_pos_embedding_forward": (c_int, [P, P, c_int, c_int, c_int, P]),
    "mi_pos_embedding_backward": (c_int, [P, P, c_int, c_int, c_int, P]),
    "mi_embedding_pos_forward": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, P]),
    "mi_embedding_pos_backward": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, P]),
    # softmax / cross-entropy
    "mi_softmax_forward": (c_int, [P, P, c_int, c_int, P]),
    "mi_cross_entropy_forward": (c_int, [P, P, P, c_int, c_int, P, P]),
    "mi_cross_entropy_forward_v2": (c_int, [P, P, P, P, P, c_int, c_int, P]),
    "mi_cross_entropy_workspace": (c_size_t, [c_int]),
    # optimizer
    "mi_scale_buffer": (c_int, [P, c_float, c_longlong, P]),
    "mi_buffer_norm_sq_acc": (c_int, [P, c_longlong, P, P]),
    "mi_compute_clip_scale": (c_int, [P, P, c_float, P]),
    "mi_adam_clipped": (c_int, [P, P, P, P, P, c_float, c_float, c_float, c_float, c_float,
                                c_float, c_float, c_longlong, P]),
    "mi_adam_update": (c_int, [P, P, P, P, c_longlong, c_float, c_float, c_float, c_float, c_int,
                               c_float, P, P, P]),
    "mi_norm_sq_workspace": (c_size_t, [c_longlong]),
    # 16-bit storage
    "mi_float_to_half": (c_int, [P, P, c_longlong, P]),
    "mi_half_to_float": (c_int, [P, P, c_longlong, P]),
    "mi_float_to_bf16": (c_int, [P, P, c_longlong, P]),
    "mi_bf16_to_float": (c_int, [P, P, c_longlong, P]),
    "mi_bias_relu_forward_to_half": (c_int, [P, P, P, c_int, c_int, P]),
    "mi_bias_gelu_forward_to_half": (c_int, [P, P, P, c_int, c_int, P]),
    "mi_bias_gelu_forward_to_bf16": (c_int, [P, P, P, c_int, c_int, P]),
    "mi_relu_backward_with_bias_backward_half_mask": (c_int, [P, P, P, P, c_int, c_int, P]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def declared_c_symbols() -> list[str]:
    """Names of every function include/mi_kernels.h declares."""
    with open(HEADERS[0]) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def last_error() -> str:
    return lib.mi_last_error().decode()


def _check(rc: int) -> None:
    if rc != MI_OK:
        raise MIError(rc, last_error())


def _ptr(x, dtype=None):
    """Device address of a torch CUDA tensor or a raw int address."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    import torch
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"expected a torch tensor or int address, got {type(x)}")
    if not x.is_cuda:
        raise ValueError("tensor must live on the GPU")
    if not x.is_contiguous():
        raise ValueError("tensor must be contiguous")
    if dtype is not None and x.dtype != dtype:
        raise ValueError(f"tensor dtype {x.dtype}, expected {dtype}")
    return x.data_ptr()


def _f(x):
    import torch
    return _ptr(x, torch.float32)


def _i(x):
    import torch
    return _ptr(x, torch.int32)


def _resolve_current_stream():
    """Returns a function that gives the raw hipStream_t of torch's current
    stream on the current device.  torch's private binding
    (_cuda_getCurrentRawStream) costs about a microsecond per call; if a torch
    release renames it, the public torch.cuda.current_stream().cuda_stream
    (a few microseconds) is used instead.  Resolved once, at import."""
    try:
        import torch
    except ImportError:
        return lambda: None
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    dev = getattr(torch._C, "_cuda_getDevice", None)
    if raw is not None and dev is not None:
        return lambda: raw(dev())
    return lambda: torch.cuda.current_stream().cuda_stream


_current_stream = _resolve_current_stream()


def _stream(stream):
    if stream is not None:
        return stream
    return _current_stream()


class Bound:
    """One C-ABI call with its arguments converted once (device addresses,
    sizes, scalars), for callers that issue the same call many times: a
    call costs the ctypes dispatch alone, not the per-call tensor checks and
    conversions of the wrapper functions.  The stream is torch's current one
    at call time unless one was given.  The tensors are kept alive with the
    binding.  Raises MIError on a non-zero status, like the wrappers."""

    def __init__(self, name, *args, stream=None):
        import torch
        fn = getattr(lib, name)
        types = _SIGS[name][1]
        if len(args) != len(types) - 1:
            raise TypeError(f"{name}: {len(types) - 1} arguments before the stream, "
                            f"got {len(args)}")
        self._keep = [a for a in args if isinstance(a, torch.Tensor)]
        conv = []
        for a, t in zip(args, types[:-1]):
            if isinstance(a, torch.Tensor):
                conv.append(c_void_p(_ptr(a)))
            else:
                conv.append(t(a) if a is not None else None)
        self._fn, self._args, self._stream = fn, tuple(conv), stream
        self.name = name

    def __call__(self):
        st = self._stream
        if st is None:
            st = _current_stream()
        rc = self._fn(*self._args, st)
        if rc != MI_OK:
            raise MIError(rc, last_error())


def bind(name, *args, stream=None) -> Bound:
    """Bound(name, *args): e.g. bind("mi_layernorm_backward", g, x, m, s, gamma,
    dx, dgamma, dbeta, rows, cols)()."""
    return Bound(name, *args, stream=stream)


# ----- runtime ----------------------------------------------------------------

def workspace_reserve(nbytes: int) -> None:
    _check(lib.mi_workspace_reserve(nbytes))


def workspace_bytes() -> int:
    return lib.mi_workspace_bytes()


def workspace_release() -> None:
    _check(lib.mi_workspace_release())


def device_sync() -> None:
    _check(lib.mi_device_sync())


# ----- LayerNorm (reference kernels.h:53-76) -----------------------------------

def layernorm_forward(x, gamma, beta, out, rows, cols, eps=1e-5, stream=None):
    _check(lib.mi_layernorm_forward(_f(x), _f(gamma), _f(beta), _f(out), rows, cols, eps,
                                    _stream(stream)))


def layernorm_forward_save(x, gamma, beta, out, mean, inv_std, rows, cols, eps=1e-5,
                           stream=None):
    _check(lib.mi_layernorm_forward_save(_f(x), _f(gamma), _f(beta), _f(out), _f(mean),
                                         _f(inv_std), rows, cols, eps, _stream(stream)))


def residual_layernorm_forward_save(a, b, gamma, beta, residual_out, out, mean, inv_std, rows,
                                    cols, eps=1e-5, stream=None):
    _check(lib.mi_residual_layernorm_forward_save(
        _f(a), _f(b), _f(gamma), _f(beta), _f(residual_out), _f(out), _f(mean), _f(inv_std),
        rows, cols, eps, _stream(stream)))


def layernorm_backward(grad_out, x, mean, inv_std, gamma, grad_x, dgamma, dbeta, rows, cols,
                       stream=None):
    _check(lib.mi_layernorm_backward(_f(grad_out), _f(x), _f(mean), _f(inv_std), _f(gamma),
                                     _f(grad_x), _f(dgamma), _f(dbeta), rows, cols,
                                     _stream(stream)))


def layernorm_backward_residual(grad_out, x, mean, inv_std, gamma, grad_residual, dgamma, dbeta,
                                rows, cols, stream=None):
    _check(lib.mi_layernorm_backward_residual(_f(grad_out), _f(x), _f(mean), _f(inv_std),
                                              _f(gamma), _f(grad_residual), _f(dgamma),
                                              _f(dbeta), rows, cols, _stream(stream)))


# Static-scratch size of mi_layernorm_backward_noalloc (MI_LN_BWD_NOALLOC_MAX_BYTES).
LN_BWD_NOALLOC_MAX_BYTES = 16 * 1024 * 1024 + 256


def layernorm_backward_noalloc(grad_out, x, mean, inv_std, gamma, grad_x, dgamma, dbeta, rows,
                               cols, stream=None):
    """layernorm_backward without any device allocation: the partial rows use
    the library's static per-device scratch (no reference counterpart)."""
    _check(lib.mi_layernorm_backward_noalloc(_f(grad_out), _f(x), _f(mean), _f(inv_std),
                                             _f(gamma), _f(grad_x), _f(dgamma), _f(dbeta), rows,
                                             cols, _stream(stream)))


# ----- residual / bias / activations (reference kernels.h:78-111) -------------

def residual_add(a, b, out, n, stream=None):
    _check(lib.mi_residual_add(_f(a), _f(b), _f(out), n, _stream(stream)))


def residual_add_with_bias(residual, x, bias, out, rows, cols, stream=None):
    _check(lib.mi_residual_add_with_bias(_f(residual), _f(x), _f(bias), _f(out), rows, cols,
                                         _stream(stream)))


def bias_add(out, bias, rows, cols, stream=None):
    _check(lib.mi_bias_add(_f(out), _f(bias), rows, cols, _stream(stream)))


def relu_forward(inp, out, n, stream=None):
    _check(lib.mi_relu_forward(_f(inp), _f(out), n, _stream(stream)))


def relu_backward(inp, grad_out, grad_in, n, stream=None):
    _check(lib.mi_relu_backward(_f(inp), _f(grad_out), _f(grad_in), n, _stream(stream)))


def bias_relu_forward(inp, bias, out, rows, cols, stream=None):
    _check(lib.mi_bias_relu_forward(_f(inp), _f(bias), _f(out), rows, cols, _stream(stream)))


def relu_backward_with_bias_backward(mask, grad_out, grad_in, dbias, rows, cols, stream=None):
    _check(lib.mi_relu_backward_with_bias_backward(_f(mask), _f(grad_out), _f(grad_in),
                                                   _f(dbias), rows, cols, _stream(stream)))


def bias_backward(grad, dbias, rows, cols, stream=None):
    _check(lib.mi_bias_backward(_f(grad), _f(dbias), rows, cols, _stream(stream)))


def bias_gelu_forward(inp, bias, out, rows, cols, stream=None):
    _check(lib.mi_bias_gelu_forward(_f(inp), _f(bias), _f(out), rows, cols, _stream(stream)))


def gelu_backward_with_bias_backward(inp, bias, grad_out, grad_in, dbias, rows, cols,
                                     stream=None):
    _check(lib.mi_gelu_backward_with_bias_backward(_f(inp), _f(bias), _f(grad_out), _f(grad_in),
                                                   _f(dbias), rows, cols, _stream(stream)))


# ----- embedding (reference kernels.h:131-138) ---------------------------------

def embedding_forward(table, tokens, out, batch_seq, dim, vocab=0, stream=None):
    _check(lib.mi_embedding_forward(_f(table), _i(tokens), _f(out), batch_seq, dim, vocab,
                                    _stream(stream)))


def embedding_backward(grad_out, tokens, grad_table, batch_seq, dim, vocab=0, stream=None):
    _check(lib.mi_embedding_backward(_f(grad_out), _i(tokens), _f(grad_table), batch_seq, dim,
                                     vocab, _stream(stream)))


def pos_embedding_forward(pos_table, embeddings, batch, seq, dim, stream=None):
    _check(lib.mi_pos_embedding_forward(_f(pos_table), _f(embeddings), batch, seq, dim,
                                        _stream(stream)))


def pos_embedding_backward(grad_out, grad_pos_table, batch, seq, dim, stream=None):
    _check(lib.mi_pos_embedding_backward(_f(grad_out), _f(grad_pos_table), batch, seq, dim,
                                         _stream(stream)))


def embedding_pos_forward(table, pos_table, tokens, out, batch, seq, dim, vocab=0, stream=None):
    _check(lib.mi_embedding_pos_forward(_f(table), _f(pos_table), _i(tokens), _f(out), batch,
                                        seq, dim, vocab, _stream(stream)))


def embedding_pos_backward(grad_out, tokens, grad_table, grad_pos_table, batch, seq, dim, vocab=0,
                           stream=None):
    """embedding_backward + pos_embedding_backward in one launch (bit-identical to the two
    calls); the reference calls them back to back at FC/src/model/transformer.cu:581-584."""
    _check(lib.mi_embedding_pos_backward(_f(grad_out), _i(tokens), _f(grad_table),
                                         _f(grad_pos_table), batch, seq, dim, vocab,
                                         _stream(stream)))


def softmax_forward(x, out, rows, cols, stream=None):
    _check(lib.mi_softmax_forward(_f(x), _f(out), rows, cols, _stream(stream)))


def cross_entropy_forward(logits, targets, grad, batch, vocab, stream=None) -> float:
    """Mean loss as a Python float (waits for the stream, as the reference's
    cross_entropy_forward returns it to the host)."""
    loss = ctypes.c_float(0.0)
    _check(lib.mi_cross_entropy_forward(_f(logits), _i(targets), _f(grad), batch, vocab,
                                        ctypes.byref(loss), _stream(stream)))
    return loss.value


def cross_entropy_forward_v2(logits, targets, grad, losses, loss_out, batch, vocab, stream=None):
    _check(lib.mi_cross_entropy_forward_v2(_f(logits), _i(targets), _f(grad), _f(losses),
                                           _f(loss_out), batch, vocab, _stream(stream)))


def scale_buffer(buf, scale, n, stream=None):
    _check(lib.mi_scale_buffer(_f(buf), scale, n, _stream(stream)))


def buffer_norm_sq_acc(buf, n, result, stream=None):
    _check(lib.mi_buffer_norm_sq_acc(_f(buf), n, _f(result), _stream(stream)))


def compute_clip_scale(norm_sq, clip_scale, max_norm, stream=None):
    _check(lib.mi_compute_clip_scale(_f(norm_sq), _f(clip_scale), max_norm, _stream(stream)))


def adam_clipped(param, grad, m, v, clip_scale, lr, beta1, beta2, eps, bc1, bc2, grad_scale, n,
                 stream=None):
    _check(lib.mi_adam_clipped(_f(param), _f(grad), _f(m), _f(v), _f(clip_scale), lr, beta1,
                               beta2, eps, bc1, bc2, grad_scale, n, _stream(stream)))


def adam_update(param, grad, m, v, n, lr, beta1, beta2, eps, step, grad_scale, norm_sq,
                clip_scale, stream=None):
    _check(lib.mi_adam_update(_f(param), _f(grad), _f(m), _f(v), n, lr, beta1, beta2, eps, step,
                              grad_scale, _f(norm_sq), _f(clip_scale), _stream(stream)))


def _h(x):
    """16-bit buffer: a torch float16 / bfloat16 tensor (or int address)."""
    import torch
    if isinstance(x, torch.Tensor) and x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"expected a float16 or bfloat16 tensor, got {x.dtype}")
    return _ptr(x)


def float_to_half(inp, out16, n, stream=None):
    _check(lib.mi_float_to_half(_f(inp), _h(out16), n, _stream(stream)))


def half_to_float(in16, out, n, stream=None):
    _check(lib.mi_half_to_float(_h(in16), _f(out), n, _stream(stream)))


def float_to_bf16(inp, out16, n, stream=None):
    _check(lib.mi_float_to_bf16(_f(inp), _h(out16), n, _stream(stream)))


def bf16_to_float(in16, out, n, stream=None):
    _check(lib.mi_bf16_to_float(_h(in16), _f(out), n, _stream(stream)))


def bias_relu_forward_to_half(inp, bias, out16, rows, cols, stream=None):
    _check(lib.mi_bias_relu_forward_to_half(_f(inp), _f(bias), _h(out16), rows, cols,
                                            _stream(stream)))


def bias_gelu_forward_to_half(inp, bias, out16, rows, cols, stream=None):
    _check(lib.mi_bias_gelu_forward_to_half(_f(inp), _f(bias), _h(out16), rows, cols,
                                            _stream(stream)))


def bias_gelu_forward_to_bf16(inp, bias, out16, rows, cols, stream=None):
    _check(lib.mi_bias_gelu_forward_to_bf16(_f(inp), _f(bias), _h(out16), rows, cols,
                                            _stream(stream)))


def relu_backward_with_bias_backward_half_mask(mask16, grad_out, grad_in, dbias, rows, cols,
                                               stream=None):
    _check(lib.mi_relu_backward_with_bias_backward_half_mask(_h(mask16), _f(grad_out),
                                                             _f(grad_in), _f(dbias), rows, cols,
                                                             _stream(stream)))
