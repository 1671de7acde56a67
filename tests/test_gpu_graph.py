"""Graph capture of the hot-path calls through the C ABI, as a caller that
captures its step (the reference's CME213_USE_CUDA_GRAPH path,
FINAL_CLEAN_CODE/src/main.cu:264-320) would: LayerNorm forward/backward,
bias+GELU forward/backward and the fused embedding forward/backward, with
the gradients cleared by fill kernels inside the graph.  Each of three
replays, with every output clobbered first and an eager step in between,
must equal the eager step bit for bit."""
import pytest
import torch

import cme213_amd as M
from gpu_util import host
from tol import assert_colsum, assert_exact

pytestmark = pytest.mark.gpu


def test_graph_replays_match_the_eager_step(dev):
    R, C, F = 2048, 768, 3072
    V, B, T = 5000, 4, 256
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2027)

    def rn(*shape, scale=1.0):
        return torch.randn(*shape, device=dev, generator=gen) * scale

    x, dy, gamma, beta = rn(R, C), rn(R, C), 1.0 + rn(C, scale=0.02), rn(C, scale=0.02)
    h, dh, bias = rn(R, F, scale=1.5), rn(R, F), rn(F, scale=0.02)
    wte, wpe, dout = rn(V, C, scale=0.02), rn(T, C, scale=0.02), rn(B * T, C)
    ids = torch.randint(0, V, (B * T,), device=dev, generator=gen, dtype=torch.int32)
    ids[:64] = 7  # a repeated id: a run of 64 rows into one table row

    y, dx = torch.empty(R, C, device=dev), torch.empty(R, C, device=dev)
    mean, rstd = torch.empty(R, device=dev), torch.empty(R, device=dev)
    dgamma, dbeta = torch.empty(C, device=dev), torch.empty(C, device=dev)
    o, gin, dbias = torch.empty(R, F, device=dev), torch.empty(R, F, device=dev), torch.empty(F, device=dev)
    emb, dwte, dwpe = torch.empty(B * T, C, device=dev), torch.empty(V, C, device=dev), torch.empty(T, C, device=dev)
    outputs = {"y": y, "mean": mean, "rstd": rstd, "dx": dx, "dgamma": dgamma, "dbeta": dbeta,
               "gelu": o, "grad_in": gin, "dbias": dbias, "emb": emb, "dwte": dwte, "dwpe": dwpe}

    def step():
        for t in (dgamma, dbeta, dbias, dwte, dwpe):  # zero_grad: fill kernels, no memset
            t.fill_(0.0)
        M.layernorm_forward_save(x, gamma, beta, y, mean, rstd, R, C, 1e-5)
        M.layernorm_backward(dy, x, mean, rstd, gamma, dx, dgamma, dbeta, R, C)
        M.bias_gelu_forward(h, bias, o, R, F)
        M.gelu_backward_with_bias_backward(h, bias, dh, gin, dbias, R, F)
        M.embedding_pos_forward(wte, wpe, ids, emb, B, T, C, V)
        M.embedding_pos_backward(dout, ids, dwte, dwpe, B, T, C, V)

    M.workspace_reserve(64 << 20)  # the reductions' workspace cannot grow during capture
    step()
    torch.cuda.synchronize()
    ref = {k: host(t) for k, t in outputs.items()}

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

    for rep in range(3):
        for t in outputs.values():
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for k, t in outputs.items():
            assert_exact(f"replay {rep} {k}", host(t), ref[k])
        step()  # eager work between replays
        torch.cuda.synchronize()
        for k, t in outputs.items():
            assert_exact(f"eager after replay {rep} {k}", host(t), ref[k])


def test_graph_replays_after_workspace_growth(dev):
    """A graph captured with workspace-using calls keeps working after an eager
    call grows the workspace: the buffer baked into the graph is retired, not
    freed, so replays neither fault nor corrupt memory handed out since."""
    R, C, F = 1024, 768, 3072
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2028)

    def rn(*shape, scale=1.0):
        return torch.randn(*shape, device=dev, generator=gen) * scale

    x, dy, gamma = rn(R, C), rn(R, C), 1.0 + rn(C, scale=0.02)
    h, dh, bias = rn(R, F, scale=1.5), rn(R, F), rn(F, scale=0.02)
    mean, rstd = torch.empty(R, device=dev), torch.empty(R, device=dev)
    M.layernorm_forward_save(x, gamma, torch.zeros(C, device=dev), torch.empty(R, C, device=dev),
                             mean, rstd, R, C, 1e-5)
    dx, gin = torch.empty(R, C, device=dev), torch.empty(R, F, device=dev)
    dgamma, dbeta, dbias = (torch.empty(C, device=dev), torch.empty(C, device=dev),
                            torch.empty(F, device=dev))
    outputs = {"dx": dx, "dgamma": dgamma, "dbeta": dbeta, "grad_in": gin, "dbias": dbias}

    def step():
        for t in (dgamma, dbeta, dbias):
            t.fill_(0.0)
        M.layernorm_backward(dy, x, mean, rstd, gamma, dx, dgamma, dbeta, R, C)
        M.gelu_backward_with_bias_backward(h, bias, dh, gin, dbias, R, F)

    step()
    torch.cuda.synchronize()
    ref = {k: host(t) for k, t in outputs.items()}
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

    # An eager call that needs more workspace than the graph was captured with.
    before = M.workspace_bytes()
    rows, cols = 64, 1 << 16
    while M.lib.mi_bias_backward_workspace(rows, cols) <= before:
        cols *= 2
    g = rn(rows, cols)
    db = torch.zeros(cols, device=dev)
    M.bias_backward(g, db, rows, cols)
    torch.cuda.synchronize()
    assert M.workspace_bytes() > before
    assert_colsum("bias_backward after growth", host(db), host(g.double().sum(0)), host(g))
    # Memory handed out after the growth must not be written by the replays.
    filler = torch.full((before // 4 + 1024,), 3.0, device=dev)

    for rep in range(3):
        for t in outputs.values():
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for k, t in outputs.items():
            assert_exact(f"replay {rep} after growth {k}", host(t), ref[k])
        step()
        torch.cuda.synchronize()
    assert bool((filler == 3.0).all())

    # Releasing the workspace (no graph left to replay) and using it again.
    del graph
    torch.cuda.synchronize()
    M.workspace_release()
    assert M.workspace_bytes() == 0
    step()
    torch.cuda.synchronize()
    for k, t in outputs.items():
        assert_exact(f"eager after release {k}", host(t), ref[k])
