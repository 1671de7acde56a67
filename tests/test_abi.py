"""CPU checks of the C ABI library: it loads without a GPU, exports every
symbol include/*.h declares, and rejects bad arguments on the host before
touching the device."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

import cme213_amd as M


def test_library_loads_and_reports_version():
    assert M.lib.mi_version().decode().startswith("cme213_amd")


def test_every_declared_c_symbol_is_exported():
    names = M.declared_c_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(M.lib, n)]
    assert not missing, missing
    # and the ctypes signature table covers them all
    assert set(names) <= set(M._SIGS), set(names) - set(M._SIGS)


@pytest.mark.skipif(shutil.which("nm") is None, reason="nm not available")
def test_every_cxx_dropin_symbol_is_exported():
    with open(M.HEADERS[1]) as f:
        text = f.read()
    declared = set(re.findall(r"^void\s+([a-z_0-9]+)\s*\(", text, re.M))
    assert {"layernorm_forward", "layernorm_backward_residual", "embedding_backward",
            "bias_gelu_forward", "gelu_backward_with_bias_backward"} <= declared
    out = subprocess.run(["nm", "-DC", "--defined-only", M.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T ([a-z_0-9]+)\(", out))
    assert declared <= exported, declared - exported


def test_host_side_argument_errors():
    lib = M.lib
    # invalid shapes are rejected before any HIP call
    assert lib.mi_layernorm_forward(None, None, None, None, -1, 768, 1e-5, None) == M.MI_ERR_INVALID_ARG
    assert "invalid shape" in M.last_error()
    assert lib.mi_layernorm_forward(None, None, None, None, 4, 0, 1e-5, None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_layernorm_backward(None, None, None, None, None, None, None, None, 8, -3,
                                     None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_bias_gelu_forward(None, None, None, -2, 8, None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_residual_add(None, None, None, -5, None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_embedding_backward(None, None, None, 16, 0, 0, None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_embedding_pos_backward(None, None, None, None, 4, 0, 64, 0,
                                         None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_embedding_pos_backward(None, None, None, None, 4, 8, 64, 0,
                                         None) == M.MI_ERR_INVALID_ARG
    assert "NULL" in M.last_error()
    # NULL pointers with a non-empty shape are rejected
    assert lib.mi_layernorm_forward_save(None, None, None, None, None, None, 4, 8, 1e-5,
                                         None) == M.MI_ERR_INVALID_ARG
    assert "NULL" in M.last_error()
    assert lib.mi_gelu_backward_with_bias_backward(None, None, None, None, None, 4, 8,
                                                   None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_softmax_forward(None, None, 4, 0, None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_cross_entropy_forward_v2(None, None, None, None, None, 4, 10,
                                           None) == M.MI_ERR_INVALID_ARG
    loss = ctypes.c_float(0)
    assert lib.mi_cross_entropy_forward(None, None, None, -1, 10, ctypes.byref(loss),
                                        None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_adam_update(None, None, None, None, 10, 1e-3, 0.9, 0.999, 1e-8, 0, 1.0, None,
                              None, None) == M.MI_ERR_INVALID_ARG
    assert lib.mi_scale_buffer(None, 2.0, -1, None) == M.MI_ERR_INVALID_ARG
    # empty inputs are a successful no-op
    assert lib.mi_layernorm_forward(None, None, None, None, 0, 768, 1e-5, None) == M.MI_OK
    assert lib.mi_residual_add(None, None, None, 0, None) == M.MI_OK
    assert lib.mi_embedding_forward(None, None, None, 0, 768, 0, None) == M.MI_OK
    assert lib.mi_embedding_pos_backward(None, None, None, None, 0, 8, 64, 0, None) == M.MI_OK
    assert lib.mi_softmax_forward(None, None, 0, 10, None) == M.MI_OK


def test_workspace_size_queries():
    # counters (256 B) + group rows + partial rows, at most 512 partial rows
    ln = M.lib.mi_layernorm_backward_workspace(8192, 768)
    assert 2 * 768 * 4 < ln <= 256 + (512 + 32) * 2 * 768 * 4 + 256
    gb = M.lib.mi_bias_backward_workspace(8192, 3072)
    assert 3072 * 4 < gb <= 256 + (512 + 32) * 3072 * 4 + 256
    assert M.lib.mi_embedding_backward_workspace(16384) == 0  # one kernel, LDS only
    assert M.lib.mi_layernorm_backward_workspace(0, 768) == 0
    assert M.lib.mi_cross_entropy_workspace(8192) >= 8192 * 4


def test_bound_call_converts_once_and_raises_on_error():
    # NULL device pointers with a valid shape: rejected on the host, no GPU call
    f = M.bind("mi_layernorm_forward", 0, 0, 0, 0, 4, 8, 1e-5, stream=0)
    with pytest.raises(M.MIError) as e:
        f()
    assert e.value.code == M.MI_ERR_INVALID_ARG and "NULL" in str(e.value)
    # an empty shape is a successful no-op, repeatably
    g = M.bind("mi_residual_add", 0, 0, 0, 0, stream=0)
    g()
    g()
    # the argument count is checked against the C signature (stream excluded)
    with pytest.raises(TypeError):
        M.bind("mi_residual_add", 0, 0, 0)


def test_noalloc_backward_rejects_oversized_shapes_on_the_host():
    # 256 partial rows of 2 * 12288 floats need 24 MiB: more than the static
    # scratch, rejected before any device call (the pointers are never used)
    rows, cols = 4096, 12288
    assert M.lib.mi_layernorm_backward_workspace(rows, cols) > M.LN_BWD_NOALLOC_MAX_BYTES
    p = 256  # a non-NULL, 16-byte aligned stand-in address
    rc = M.lib.mi_layernorm_backward_noalloc(p, p, p, p, p, p, p, p, rows, cols, None)
    assert rc == M.MI_ERR_INVALID_ARG and "scratch" in M.last_error()
    # the header's size and the Python constant agree
    with open(M.HEADERS[0]) as f:
        hdr = f.read()
    assert "#define MI_LN_BWD_NOALLOC_MAX_BYTES ((size_t)16 * 1024 * 1024 + 256)" in hdr
    assert M.LN_BWD_NOALLOC_MAX_BYTES == 16 * 1024 * 1024 + 256
