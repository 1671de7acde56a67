"""GPU parity of the optimizer step over the flat parameter buffer
(FINAL_CLEAN_CODE/src/kernels/activations.cu:349-392,
src/model/transformer.cu:598-636) against the CPU oracle:
  * scale_buffer: bit-exact (one multiply);
  * buffer_norm_sq_acc: the `+=` contract, within 1e-5 relative of the
    float64 sum of squares (the reference's float atomics fix no order),
    and bitwise repeatable;
  * compute_clip_scale: bit-exact given the same norm²;
  * clipped Adam: bit-exact against the oracle's statement of
    adam_clipped_kernel given the same clip scale (the kernel evaluates the
    arithmetic as written, without FMA contraction);
  * adam_update (update_adam's sequence): norm², clip scale and step.
Sizes include n % 4 != 0 and a misaligned base (scalar path) and
GPT-2-small's parameter count."""
import numpy as np
import pytest
import torch

import cme213_amd as M
import oracle as O
from gpu_util import dev_t, host, note
from tol import assert_exact

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 1000, 1001, 65536 * 4 + 3, 4_000_000]


def _vecs(n, seed):
    r = np.random.default_rng(seed)
    p = r.standard_normal(n).astype(np.float32)
    g = (2 * r.standard_normal(n)).astype(np.float32)
    m = (0.1 * r.standard_normal(n)).astype(np.float32)
    v = (0.01 * r.random(n)).astype(np.float32)
    return p, g, m, v


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("offset", [0, 1])
def test_scale_norm_clip_adam(dev, n, offset):
    note(f"optim n={n} offset={offset}")
    p, g, m, v = _vecs(n, n + offset)
    # an offset of one float gives a base that is not 16-byte aligned
    def dev_off(a):
        buf = torch.zeros(a.size + offset, device="cuda")
        buf[offset:] = dev_t(a)
        return buf[offset:]
    P_, G_, Mm, V_ = dev_off(p), dev_off(g), dev_off(m), dev_off(v)

    S = dev_off(g)
    M.scale_buffer(S, 0.125, n)
    assert_exact("scale_buffer", host(S), O.scale_buffer(g, 0.125))

    res = torch.full((1,), 5.0, device="cuda")
    M.buffer_norm_sq_acc(G_, n, res)
    got = float(host(res)[0])
    ref = 5.0 + O.sumsq_f64(g)
    assert abs(got - ref) <= 1e-5 * ref, (got, ref)
    again = torch.full((1,), 5.0, device="cuda")
    M.buffer_norm_sq_acc(G_, n, again)
    assert_exact("norm² repeat", host(again), host(res))

    clip = torch.empty(1, device="cuda")
    M.compute_clip_scale(res, clip, 3.0)
    assert_exact("clip scale", host(clip), np.float32(O.clip_scale(np.float32(got), 3.0)).reshape(1))

    lr, b1, b2, eps, gs = 3e-4, 0.9, 0.999, 1e-8, 0.5
    bc1, bc2 = O.adam_bias_corrections(b1, b2, 3)
    M.adam_clipped(P_, G_, Mm, V_, clip, lr, b1, b2, eps, bc1, bc2, gs, n)
    po, mo, vo = O.adam_clipped(p, g, m, v, float(host(clip)[0]), lr, b1, b2, eps, bc1, bc2, gs)
    assert_exact("adam m", host(Mm), mo)
    assert_exact("adam v", host(V_), vo)
    assert_exact("adam param", host(P_), po)


@pytest.mark.parametrize("step", [1, 2, 10])
def test_adam_update_sequence(dev, step):
    n = 3_000_001
    note(f"adam_update n={n} step={step}")
    p, g, m, v = _vecs(n, 100 + step)
    if step == 1:
        m[:] = 0
        v[:] = 0
    P_, G_, Mm, V_ = dev_t(p), dev_t(g), dev_t(m), dev_t(v)
    norm_sq, clip = torch.full((1,), 123.0, device="cuda"), torch.empty(1, device="cuda")
    lr, b1, b2, eps, gs = 1e-3, 0.9, 0.95, 1e-8, 1.0 / 64
    M.adam_update(P_, G_, Mm, V_, n, lr, b1, b2, eps, step, gs, norm_sq, clip)
    got = float(host(norm_sq)[0])
    ref = O.sumsq_f64(g)          # overwritten, not accumulated
    assert abs(got - ref) <= 1e-5 * ref, (got, ref)
    c = O.clip_scale(np.float32(got), 64.0)
    assert_exact("clip", host(clip), np.float32(c).reshape(1))
    bc1, bc2 = O.adam_bias_corrections(b1, b2, step)
    po, mo, vo = O.adam_clipped(p, g, m, v, c, lr, b1, b2, eps, bc1, bc2, gs)
    assert_exact("m", host(Mm), mo)
    assert_exact("v", host(V_), vo)
    assert_exact("param", host(P_), po)


def test_gpt2_small_parameter_count(dev):
    n = 124_439_808  # GPT-2 small
    note(f"adam_update n={n}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    P_ = torch.randn(n, device="cuda", generator=gen)
    G_ = torch.randn(n, device="cuda", generator=gen) * 1e-3
    Mm = torch.zeros(n, device="cuda")
    V_ = torch.zeros(n, device="cuda")
    p, g = host(P_), host(G_)
    norm_sq, clip = torch.empty(1, device="cuda"), torch.empty(1, device="cuda")
    M.adam_update(P_, G_, Mm, V_, n, 3e-4, 0.9, 0.999, 1e-8, 1, 1.0, norm_sq, clip)
    got = float(host(norm_sq)[0])
    ref = O.sumsq_f64(g)
    assert abs(got - ref) <= 1e-5 * ref, (got, ref)
    bc1, bc2 = O.adam_bias_corrections(0.9, 0.999, 1)
    z = np.zeros(n, np.float32)
    po, mo, vo = O.adam_clipped(p, g, z, z, float(host(clip)[0]), 3e-4, 0.9, 0.999, 1e-8, bc1,
                                bc2, 1.0)
    assert_exact("param", host(P_), po)
    assert_exact("m", host(Mm), mo)


def test_adam_past_one_vector_per_thread(dev):
    # 2^25 + 1 vectors: one more than the one-vector-per-thread grid covers,
    # so the last vector goes through the kernel's grid-stride loop
    n = (1 << 27) + 4
    note(f"adam_clipped n={n}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    P_ = torch.randn(n, device="cuda", generator=gen)
    G_ = torch.randn(n, device="cuda", generator=gen)
    Mm = torch.randn(n, device="cuda", generator=gen) * 0.1
    V_ = torch.rand(n, device="cuda", generator=gen) * 0.01
    p, g, m, v = host(P_), host(G_), host(Mm), host(V_)
    clip = torch.full((1,), 0.75, device="cuda")
    bc1, bc2 = O.adam_bias_corrections(0.9, 0.999, 4)
    M.adam_clipped(P_, G_, Mm, V_, clip, 3e-4, 0.9, 0.999, 1e-8, bc1, bc2, 1.0, n)
    po, mo, vo = O.adam_clipped(p, g, m, v, 0.75, 3e-4, 0.9, 0.999, 1e-8, bc1, bc2, 1.0)
    assert_exact("param", host(P_), po)
    assert_exact("m", host(Mm), mo)
    assert_exact("v", host(V_), vo)
