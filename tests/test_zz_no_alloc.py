"""The allocation-free LayerNorm backward (mi_layernorm_backward_noalloc)
against mi_layernorm_backward, through the C ABI: two calls in a row, the
second on a smaller input, each bit-identical to the workspace entry point
(same kernels, same partial-row count, so the same summation order), and dx
also held to the oracle's tolerance.  The second call reuses the static
scratch the first one filled, so a stale partial row would show up here."""
import numpy as np
import pytest
import torch

import cme213_amd as M
import oracle as O
from gpu_util import dev_t, host, ln_inputs, note
from tol import assert_bwd, assert_exact

pytestmark = pytest.mark.gpu


def _run(fn, g, x, m, s, gamma, dg0, db0, rows, cols):
    DX = torch.full((rows, cols), float("nan"), device="cuda:0")
    DG, DB = dev_t(dg0), dev_t(db0)
    fn(dev_t(g), dev_t(x), dev_t(m), dev_t(s), dev_t(gamma), DX, DG, DB, rows, cols)
    return host(DX), host(DG), host(DB)


@pytest.mark.parametrize("shapes", [((8192, 768), (1000, 768)), ((4096, 1600), (333, 1024)),
                                    ((2048, 4096), (37, 33))])
def test_noalloc_matches_workspace_entry_point(dev, shapes):
    for i, (rows, cols) in enumerate(shapes):
        note(f"layernorm_backward_noalloc call {i} rows={rows} cols={cols}")
        assert M.lib.mi_layernorm_backward_workspace(rows, cols) <= M.LN_BWD_NOALLOC_MAX_BYTES
        x, gamma, _, g = ln_inputs(rows, cols, 900 + i)
        _, m, s = O.layernorm_forward(x, gamma, np.zeros(cols, np.float32))
        r = np.random.default_rng(i)
        dg0 = r.standard_normal(cols).astype(np.float32)
        db0 = r.standard_normal(cols).astype(np.float32)
        ref = _run(M.layernorm_backward, g, x, m, s, gamma, dg0, db0, rows, cols)
        got = _run(M.layernorm_backward_noalloc, g, x, m, s, gamma, dg0, db0, rows, cols)
        for name, a, b in zip(("dx", "dgamma", "dbeta"), got, ref):
            assert_exact(f"noalloc {name} [{rows},{cols}]", a, b)
        dx_o, _, _ = O.layernorm_backward(g, x, m, s, gamma)
        assert_bwd(f"noalloc dx vs oracle [{rows},{cols}]", got[0], dx_o)


def test_noalloc_rejects_shapes_beyond_the_scratch(dev):
    rows, cols = 4096, 12288  # 256 partial rows of 2 * 12288 floats: 24 MiB
    need = M.lib.mi_layernorm_backward_workspace(rows, cols)
    assert need > M.LN_BWD_NOALLOC_MAX_BYTES
    t = torch.zeros(8, device="cuda:0")
    p = t.data_ptr()
    rc = M.lib.mi_layernorm_backward_noalloc(p, p, p, p, p, p, p, p, rows, cols, None)
    assert rc == M.MI_ERR_INVALID_ARG
    assert "scratch" in M.last_error()
