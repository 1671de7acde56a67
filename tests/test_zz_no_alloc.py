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


def test_noalloc_uses_no_workspace_and_replays_in_a_graph(dev):
    """The entry point's defining property: with the library workspace
    released (0 bytes), an eager call and a graph capture of the call leave
    it at 0 bytes (no allocation, no use of the workspace), and every replay
    of the graph, with eager work between replays, equals the eager result
    bit for bit."""
    rows, cols = 4096, 768
    x, gamma, _, g = ln_inputs(rows, cols, 950)
    _, m, s = O.layernorm_forward(x, gamma, np.zeros(cols, np.float32))
    G, X, Mn, Rs, Gm = dev_t(g), dev_t(x), dev_t(m), dev_t(s), dev_t(gamma)
    DX = torch.empty(rows, cols, device=dev)
    DG, DB = torch.empty(cols, device=dev), torch.empty(cols, device=dev)

    def step():
        DG.fill_(0.0)  # zero_grad by fill kernels inside the graph (no memset node)
        DB.fill_(0.0)
        M.layernorm_backward_noalloc(G, X, Mn, Rs, Gm, DX, DG, DB, rows, cols)

    M.workspace_release()
    assert M.workspace_bytes() == 0
    note("layernorm_backward_noalloc eager, workspace released")
    step()
    torch.cuda.synchronize()
    assert M.workspace_bytes() == 0
    ref = [host(t) for t in (DX, DG, DB)]
    want = _run(M.layernorm_backward, g, x, m, s, gamma, np.zeros(cols, np.float32),
                np.zeros(cols, np.float32), rows, cols)
    for name, a, b in zip(("dx", "dgamma", "dbeta"), ref, want):
        assert_exact(f"noalloc eager {name}", a, b)
    # the workspace entry point just grew the workspace; release it again
    M.workspace_release()
    assert M.workspace_bytes() == 0

    note("layernorm_backward_noalloc under graph capture, no workspace reserved")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    assert M.workspace_bytes() == 0
    for rep in range(3):
        for t in (DX, DG, DB):
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name, t, r in zip(("dx", "dgamma", "dbeta"), (DX, DG, DB), ref):
            assert_exact(f"replay {rep} {name}", host(t), r)
        step()  # eager work between replays
        torch.cuda.synchronize()
        for name, t, r in zip(("dx", "dgamma", "dbeta"), (DX, DG, DB), ref):
            assert_exact(f"eager after replay {rep} {name}", host(t), r)
    assert M.workspace_bytes() == 0
    del graph
    torch.cuda.synchronize()
