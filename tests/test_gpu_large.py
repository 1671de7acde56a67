"""Tensors past 2^31 elements, through the C ABI.

The reference's sizes are `int` rows and columns (FC/include/kernels.h:53-92),
so rows * cols can pass 2^31 elements; on a 288 GB device such tensors are
ordinary.  Every kernel family runs once at such a size:
  * rows straddling element 2^31 (and 2^32, 2^33 where the tensor reaches
    them), plus the first and last rows, against the CPU oracle on those
    rows (the operations are row-local);
  * the whole tensor on the device against float64 evaluations of the same
    formulas at the stated tolerances (tests/tol.py), outputs pre-filled
    with NaN so that an element no kernel wrote fails;
  * gathers, selects and single adds bit for bit, and the embedding
    scatter-add with integer-valued gradients, whose sums are exact in any
    order, bit for bit against float64 sums;
  * the bias+GELU forward, bias add and ReLU also past 2^31 16-byte vectors,
    where the broadcast kernels leave their 32-bit flat walk for the row
    bands, and bias add just below 2^32 vectors, where a 32-bit walk would
    wrap.
About 115 GB of device memory at the peak (the GELU test); each test checks
the free memory first and releases what it allocated."""
import gc

import numpy as np
import pytest
import torch

import cme213_amd as M
import oracle as O
from gpu_util import host, note
from tol import (BWD_ATOL, BWD_RTOL, COL_RTOL, FWD_ATOL, FWD_RTOL, assert_bwd,
                 assert_bwd_within_oracle_error, assert_exact, assert_fwd,
                 assert_fwd_within_oracle_error)

pytestmark = pytest.mark.gpu

E31 = 1 << 31
EPS = float(np.float32(1e-5))
K0 = 0.79788456080286535587989211986876  # sqrt(2/pi)
K1 = 0.044715


@pytest.fixture(autouse=True)
def _release():
    yield
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _need(gib):
    free, _ = torch.cuda.mem_get_info()
    if free < gib * (1 << 30):
        pytest.skip(f"needs {gib} GiB of free device memory, {free / (1 << 30):.0f} GiB free")


def _gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def _nan(*shape):
    return torch.full(shape, float("nan"), device="cuda")


def _chunks(n, step):
    for a in range(0, n, step):
        yield a, min(n, a + step)


def _probe_rows(rows, cols):
    """First two rows, the rows around each element 2^31 * k inside the
    tensor, and the last two rows."""
    out = {0, 1, rows - 2, rows - 1}
    k = 1
    while k * E31 < rows * cols:
        b = k * E31 // cols
        out.update({b - 1, b, b + 1})
        k *= 2
    return sorted(r for r in out if 0 <= r < rows)


def _close(name, got, ref, bound, row0):
    """|got - ref| <= bound on the device; NaN fails."""
    err = (got.double() - ref).abs()
    ok = err <= bound
    if not bool(ok.all()):
        bad = ~ok
        k = int(torch.nonzero(bad.flatten())[0])
        raise AssertionError(
            f"{name}: {int(bad.sum())} of {bad.numel()} elements out of tolerance in the chunk "
            f"from row {row0}; first at flat index {k}: got {got.flatten()[k].item()!r} "
            f"ref {ref.flatten()[k].item()!r}")


def _same(name, got, ref, row0):
    eq = got.contiguous().view(torch.int32) == ref.contiguous().view(torch.int32)
    if not bool(eq.all()):
        k = int(torch.nonzero(~eq.flatten())[0])
        raise AssertionError(
            f"{name}: {int((~eq).sum())} elements differ bitwise in the chunk from row {row0}; "
            f"first at flat index {k}: got {got.flatten()[k].item()!r} "
            f"ref {ref.flatten()[k].item()!r}")


def _fwd_bound(ref):
    return FWD_ATOL + FWD_RTOL * ref.abs()


def _bwd_bound(ref):
    s = max(1.0, float(torch.sqrt((ref * ref).mean())))
    return BWD_ATOL * s + BWD_RTOL * ref.abs()


def test_layernorm_past_2_31_elements(dev):
    R, C = (1 << 21) + 37, 1024                       # 2,147,521,536 elements
    _need(56)
    note(f"large layernorm rows={R} cols={C}")
    gen = _gen(31)
    x = torch.randn(R, C, device=dev, generator=gen)
    dy = torch.randn(R, C, device=dev, generator=gen)
    gamma = 1.0 + 0.02 * torch.randn(C, device=dev, generator=gen)
    beta = 0.02 * torch.randn(C, device=dev, generator=gen)
    y, mean, rstd = _nan(R, C), _nan(R), _nan(R)
    M.layernorm_forward_save(x, gamma, beta, y, mean, rstd, R, C, 1e-5)
    dx = _nan(R, C)
    dg = torch.full((C,), 0.5, device=dev)
    db = torch.full((C,), -0.25, device=dev)
    M.layernorm_backward(dy, x, mean, rstd, gamma, dx, dg, db, R, C)
    torch.cuda.synchronize()

    idx = torch.tensor(_probe_rows(R, C), device=dev)
    xs, gs, gh, bh = host(x[idx]), host(dy[idx]), host(gamma), host(beta)
    y_o, m_o, s_o = O.layernorm_forward(xs, gh, bh)
    assert_fwd("y probe rows", host(y[idx]), y_o)
    assert_fwd("mean probe rows", host(mean[idx]), m_o)
    assert_fwd("rstd probe rows", host(rstd[idx]), s_o)
    dx_o, _, _ = O.layernorm_backward(gs, xs, host(mean[idx]), host(rstd[idx]), gh)
    assert_bwd("dx probe rows", host(dx[idx]), dx_o)

    g64, b64 = gamma.double(), beta.double()
    sg = torch.zeros(C, dtype=torch.float64, device=dev)
    sb, qg, qb = torch.zeros_like(sg), torch.zeros_like(sg), torch.zeros_like(sg)
    for a, b in _chunks(R, 1 << 17):
        x64, d64 = x[a:b].double(), dy[a:b].double()
        mu = x64.mean(1, keepdim=True)
        xc = x64 - mu
        rs = 1.0 / torch.sqrt((xc * xc).mean(1, keepdim=True) + EPS)
        _close("mean", mean[a:b], mu[:, 0], _fwd_bound(mu[:, 0]), a)
        _close("rstd", rstd[a:b], rs[:, 0], _fwd_bound(rs[:, 0]), a)
        ref = xc * rs * g64 + b64
        _close("y", y[a:b], ref, _fwd_bound(ref), a)
        # backward from the kernel's saved statistics, as the kernel computes it
        xh = (x64 - mean[a:b, None].double()) * rstd[a:b, None].double()
        gg = d64 * g64
        ref = rstd[a:b, None].double() * (gg - gg.mean(1, keepdim=True)
                                          - xh * (gg * xh).mean(1, keepdim=True))
        _close("dx", dx[a:b], ref, _bwd_bound(ref), a)
        t = d64 * xh
        sg += t.sum(0)
        qg += (t * t).sum(0)
        sb += d64.sum(0)
        qb += (d64 * d64).sum(0)
    ref_g, ref_b = sg + 0.5, sb - 0.25
    _close("dgamma", dg, ref_g, COL_RTOL * (ref_g.abs() + qg.sqrt()), 0)
    _close("dbeta", db, ref_b, COL_RTOL * (ref_b.abs() + qb.sqrt()), 0)


def _gelu64(u):
    return u / (1.0 + torch.exp(-2.0 * K0 * (u + K1 * u * u * u)))


def _gelu_grad64(u):
    t = torch.tanh(K0 * (u + K1 * u * u * u))
    return 0.5 * (1.0 + t) + 0.5 * u * (1.0 - t * t) * K0 * (1.0 + 3.0 * K1 * u * u)


def test_bias_gelu_relu_bias_add_past_2_31_vectors(dev):
    F = 3072
    R = (1 << 33) // F + 6                    # 8,589,950,976 elements: 2^31 + 4096 vectors
    n = R * F
    _need(130)
    note(f"large bias+gelu rows={R} cols={F}")
    gen = _gen(33)
    h = torch.randn(R, F, device=dev, generator=gen).mul_(1.5)
    bias = 0.02 * torch.randn(F, device=dev, generator=gen)
    out = _nan(R, F)
    M.bias_gelu_forward(h, bias, out, R, F)
    torch.cuda.synchronize()

    idx = torch.tensor(_probe_rows(R, F), device=dev)
    hs, bh = host(h[idx]), host(bias)
    y64 = O.bias_gelu_forward_f64(hs, bh)
    ys = host(out[idx])
    assert_fwd("gelu probe rows vs f64", ys, y64)
    assert_fwd_within_oracle_error("gelu probe rows vs float oracle", ys,
                                   O.bias_gelu_forward(hs, bh), y64)
    b64 = bias.double()
    step = 1 << 16
    for a, b in _chunks(R, step):
        ref = _gelu64(h[a:b].double() + b64)
        _close("gelu y", out[a:b], ref, _fwd_bound(ref), a)

    out.fill_(float("nan"))
    M.relu_forward(h, out, n)
    torch.cuda.synchronize()
    for a, b in _chunks(R, step):
        hc = h[a:b]
        _same("relu", out[a:b], torch.where(hc > 0, hc, torch.zeros_like(hc)), a)
    M.bias_add(out, bias, R, F)
    torch.cuda.synchronize()
    for a, b in _chunks(R, step):
        hc = h[a:b]
        _same("bias_add", out[a:b], torch.where(hc > 0, hc, torch.zeros_like(hc)) + bias, a)
    del out
    torch.cuda.empty_cache()

    dh = torch.randn(R, F, device=dev, generator=gen)
    gin = _nan(R, F)
    dbias = torch.full((F,), 0.125, device=dev)
    M.gelu_backward_with_bias_backward(h, bias, dh, gin, dbias, R, F)
    torch.cuda.synchronize()
    gs = host(dh[idx])
    gin64, _ = O.gelu_backward_with_bias_backward_f64(hs, bh, gs)
    gin_o, _ = O.gelu_backward_with_bias_backward(hs, bh, gs)
    gi = host(gin[idx])
    assert_bwd("gelu grad_in probe rows vs f64", gi, gin64)
    assert_bwd_within_oracle_error("gelu grad_in probe rows vs float oracle", gi, gin_o, gin64)

    s_sum = torch.zeros(F, dtype=torch.float64, device=dev)
    s_sq = torch.zeros_like(s_sum)
    s_all = 0.0
    for a, b in _chunks(R, step):
        u = (h[a:b] + bias).double()             # the float sum, widened
        ref = dh[a:b].double() * _gelu_grad64(u)
        _close("gelu grad_in", gin[a:b], ref, _bwd_bound(ref), a)
        s_sum += ref.sum(0)
        s_sq += (ref * ref).sum(0)
        s_all += float((ref * ref).sum())
    ref_db = s_sum + 0.125
    s = max(1.0, (s_all / n) ** 0.5)
    bound = COL_RTOL * (ref_db.abs() + s_sq.sqrt()) + BWD_ATOL * s * R ** 0.5
    _close("gelu dbias", dbias, ref_db, bound, 0)


def test_bias_add_just_below_2_32_vectors(dev):
    # 2^32 - 1024 vectors: a 32-bit index walk with a 4M-thread stride would
    # wrap past 2^32 here and restart; the broadcast kernels take the row
    # bands above 2^31 vectors
    F = 4096
    R = (1 << 32) // (F // 4) - 1                 # 4,294,966,272 vectors, 68.7 GB
    _need(80)
    note(f"large bias_add rows={R} cols={F}")
    gen = _gen(34)
    bias = 0.02 * torch.randn(F, device=dev, generator=gen)
    out = torch.zeros(R, F, device=dev)
    M.bias_add(out, bias, R, F)
    torch.cuda.synchronize()
    ref = torch.zeros(1, F, device=dev) + bias
    for a, b in _chunks(R, 1 << 16):
        _same("bias_add", out[a:b], ref.expand(b - a, F), a)


def test_embedding_past_2_31_elements(dev):
    B, T, D, V = 2049, 1024, 1024, 50257          # 2,148,532,224 output elements
    BT = B * T
    _need(40)
    note(f"large embedding batch={B} seq={T} dim={D} vocab={V}")
    gen = _gen(35)
    wte = 0.02 * torch.randn(V, D, device=dev, generator=gen)
    wpe = 0.02 * torch.randn(T, D, device=dev, generator=gen)
    ids = torch.randint(0, V, (BT,), device=dev, generator=gen, dtype=torch.int32)
    ids[5000:13000] = 7                           # one long run into table row 7
    out = _nan(BT, D)
    M.embedding_pos_forward(wte, wpe, ids, out, B, T, D, V)
    torch.cuda.synchronize()

    th, ph = host(wte), host(wpe)
    for bb in sorted({0, E31 // D // T, B - 1}):
        sl = slice(bb * T, (bb + 1) * T)
        ref = O.pos_embedding_forward(ph, O.embedding_forward(th, host(ids[sl])), 1, T)
        assert_exact(f"embedding forward, batch row {bb}", host(out[sl]), ref)
    step = 1 << 17
    for a, b in _chunks(BT, step):
        pos = torch.arange(a, b, device=dev) % T
        _same("embedding forward", out[a:b], wte[ids[a:b].long()] + wpe[pos], a)
    del out

    # integer-valued gradients: every sum below is exact in any order
    dout = torch.randint(-15, 16, (BT, D), device=dev, generator=gen, dtype=torch.float32)
    init_t = torch.randint(-2, 3, (V, D), device=dev, generator=gen, dtype=torch.float32)
    init_p = torch.randint(-2, 3, (T, D), device=dev, generator=gen, dtype=torch.float32)
    dwte, dwpe = init_t.clone(), init_p.clone()
    M.embedding_pos_backward(dout, ids, dwte, dwpe, B, T, D, V)
    dwte2, dwpe2 = init_t.clone(), init_p.clone()
    M.embedding_backward(dout, ids, dwte2, BT, D, V)
    M.pos_embedding_backward(dout, dwpe2, B, T, D)
    torch.cuda.synchronize()

    ref_t = init_t.double()
    ref_p = init_p.double()
    for a, b in _chunks(BT, step):
        ref_t.index_add_(0, ids[a:b].long(), dout[a:b].double())
    for bb in range(B):
        ref_p += dout[bb * T:(bb + 1) * T].double()
    ref_t, ref_p = ref_t.float(), ref_p.float()
    _same("fused backward dwte", dwte, ref_t, 0)
    _same("fused backward dwpe", dwpe, ref_p, 0)
    _same("embedding_backward dwte", dwte2, ref_t, 0)
    _same("pos_embedding_backward dwpe", dwpe2, ref_p, 0)


def test_softmax_cross_entropy_past_2_31_elements(dev):
    R, V = E31 // 50257 + 3, 50257                # 2,147,682,638 elements
    _need(40)
    note(f"large softmax / cross-entropy rows={R} cols={V}")
    gen = _gen(37)
    x = torch.randn(R, V, device=dev, generator=gen).mul_(3.0)
    t = torch.randint(0, V, (R,), device=dev, generator=gen, dtype=torch.int32)
    grad, losses, lout = _nan(R, V), _nan(R), _nan(1)
    M.cross_entropy_forward_v2(x, t, grad, losses, lout, R, V)
    y = _nan(R, V)
    M.softmax_forward(x, y, R, V)
    torch.cuda.synchronize()

    idx = torch.tensor(_probe_rows(R, V), device=dev)
    xs, ts = host(x[idx]), host(t[idx])
    lr, gr = O.cross_entropy_rows(xs, ts, 1.0 / R)
    assert_fwd("per-row losses, probe rows", host(losses[idx]), lr)
    assert_bwd("grad, probe rows", host(grad[idx]), gr)
    assert_fwd_within_oracle_error("softmax, probe rows", host(y[idx]), O.softmax_forward(xs),
                                   O.softmax_forward_f64(xs))

    scale = 1.0 / R
    tl = t.long()
    for a, b in _chunks(R, 2048):
        x64 = x[a:b].double()
        p = torch.softmax(x64, dim=1)
        _close("softmax", y[a:b], p, _fwd_bound(p), a)
        pt = p.gather(1, tl[a:b, None])[:, 0]
        l64 = -torch.log(pt)
        # the kernel's loss is -log(p[t] + 1e-9): allow 1e-9 / p[t] more
        _close("losses", losses[a:b], l64, FWD_ATOL + FWD_RTOL * l64.abs() + 1.01e-9 / pt, a)
        g64 = p.scatter_add(1, tl[a:b, None], -torch.ones(b - a, 1, dtype=torch.float64,
                                                          device=dev)) * scale
        _close("grad", grad[a:b], g64, 1e-5 * g64.abs() + 1e-6 * scale, a)
    assert_fwd("mean loss", host(lout)[0], np.float32(float(losses.double().mean())))


def test_norm_clip_adam_past_2_31_elements(dev):
    n = E31 + 3                                   # n % 4 != 0: the scalar path, 64-bit walk
    _need(80)
    note(f"large norm / clip / adam n={n}")
    gen = _gen(39)
    p = torch.randn(n, device=dev, generator=gen)
    g = 2.0 * torch.randn(n, device=dev, generator=gen)
    m = 0.1 * torch.randn(n, device=dev, generator=gen)
    v = 0.01 * torch.rand(n, device=dev, generator=gen)
    p0, m0, v0 = p.clone(), m.clone(), v.clone()
    norm_sq = torch.full((1,), 5.0, device=dev)
    M.buffer_norm_sq_acc(g, n, norm_sq)
    ref = 5.0
    for a, b in _chunks(n, 1 << 28):
        gc64 = g[a:b].double()
        ref += float((gc64 * gc64).sum())
    got = float(host(norm_sq)[0])
    assert abs(got - ref) <= 1e-5 * ref, (got, ref)

    clip = torch.empty(1, device=dev)
    M.compute_clip_scale(norm_sq, clip, 3.0)
    lr, b1, b2, eps, gsc = 3e-4, 0.9, 0.999, 1e-8, 0.5
    bc1, bc2 = O.adam_bias_corrections(b1, b2, 3)
    M.adam_clipped(p, g, m, v, clip, lr, b1, b2, eps, bc1, bc2, gsc, n)
    torch.cuda.synchronize()
    c = float(host(clip)[0])

    for a, b in [(0, 4096), (E31 - 4096, E31 + 3)]:
        po, mo, vo = O.adam_clipped(host(p0[a:b]), host(g[a:b]), host(m0[a:b]), host(v0[a:b]),
                                    c, lr, b1, b2, eps, bc1, bc2, gsc)
        assert_exact(f"adam param [{a}, {b})", host(p[a:b]), po)
        assert_exact(f"adam m [{a}, {b})", host(m[a:b]), mo)
        assert_exact(f"adam v [{a}, {b})", host(v[a:b]), vo)

    # whole buffer: m and v as float32 products and sums, each rounded (the
    # kernel's statement order), bit for bit; the parameter within the
    # forward tolerance of float64 (an element left unchanged misses by
    # about lr)
    f = lambda s: torch.tensor(np.float32(s), device=dev)  # noqa: E731
    B1, B2, OB1, OB2 = f(b1), f(b2), f(np.float32(1) - np.float32(b1)), f(np.float32(1) - np.float32(b2))
    GS, CL = f(gsc), clip[0]
    for a, b in _chunks(n, 1 << 28):
        gg = g[a:b] * GS * CL
        mi = B1 * m0[a:b] + OB1 * gg
        vi = B2 * v0[a:b] + OB2 * gg * gg
        _same("adam m", m[a:b], mi, a)
        _same("adam v", v[a:b], vi, a)
        ref = p0[a:b].double() - lr * (mi.double() / bc1) / (torch.sqrt(vi.double() / bc2) + eps)
        _close("adam param", p[a:b], ref, _fwd_bound(ref), a)
