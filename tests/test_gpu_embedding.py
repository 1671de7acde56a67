"""GPU parity of the embedding kernels against the CPU oracle (restating
NC/tests/test_embedding.cu:16-41 and FC/src/kernels/embedding.cu:61-70).
Forward and backward are bit-exact: the gather is a copy plus one add, and
the backward accumulates every table row in increasing token position, the
order of the CPU loop."""
import numpy as np
import pytest
import torch

import cme213_amd as M
import oracle as O
from gpu_util import dev_t, host, note
from tol import assert_exact

pytestmark = pytest.mark.gpu


def emb_inputs(V, D, B, T, seed, vocab_ids=None):
    r = np.random.default_rng(seed)
    wte = (0.02 * r.standard_normal((V, D))).astype(np.float32)
    wpe = (0.02 * r.standard_normal((T, D))).astype(np.float32)
    ids = r.integers(0, vocab_ids or V, B * T).astype(np.int32)
    g = r.standard_normal((B * T, D), dtype=np.float32)
    return wte, wpe, ids, g


def test_reference_embedding_test_case(dev):
    # NC/tests/test_embedding.cu:46-59: V=512, D=128, B=16, T=32, srand(42)
    V, D, B, T = 512, 128, 16, 32
    BT = B * T
    O.lib().orc_srand(42)
    table = np.empty(V * D, np.float32)
    O.lib().orc_fill_rand_unit(O._p(table), table.size)
    tokens = np.empty(BT, np.int32)
    O.lib().orc_fill_rand_tokens(O._p(tokens), BT, V)
    g = np.empty(BT * D, np.float32)
    O.lib().orc_fill_rand_unit(O._p(g), g.size)
    pos = np.empty(T * D, np.float32)
    O.lib().orc_fill_rand_unit(O._p(pos), pos.size)
    table, g, pos = table.reshape(V, D), g.reshape(BT, D), pos.reshape(T, D)

    Tb, Tk = dev_t(table), dev_t(tokens)
    out = torch.empty(BT, D, device=dev)
    M.embedding_forward(Tb, Tk, out, BT, D)
    ref = O.embedding_forward(table, tokens)
    assert_exact("embedding_forward", host(out), ref)
    gt = torch.zeros(V, D, device=dev)
    M.embedding_backward(dev_t(g), Tk, gt, BT, D)
    assert_exact("embedding_backward", host(gt),
                 O.embedding_backward(g, tokens, np.zeros((V, D), np.float32)))
    M.pos_embedding_forward(dev_t(pos), out, B, T, D)
    assert_exact("pos_embedding_forward", host(out), O.pos_embedding_forward(pos, ref, B, T))


@pytest.mark.parametrize("V,D,B,T,vocab_arg", [
    (50257, 768, 16, 1024, 50257),
    (50257, 768, 16, 1024, 0),       # ids trusted (no vocabulary bound)
    (1000, 100, 3, 333, 1000),       # D % 4 != 0, ragged last id group
    (7, 64, 2, 4, 7),                # tiny vocabulary, one owning workgroup, long runs
    (70000, 16, 1, 1, 70000),        # one token
    # more than 16384 tokens: several passes over the ids per workgroup
    (50257, 64, 33, 1000, 50257),
    (300, 32, 1, 16385, 300),        # one token into the second pass, long runs
    (70000, 16, 2, 9000, 0),         # trusted ids, 18000 tokens
    (2000, 1600, 2, 500, 2000),      # GPT-2-XL width: 4 vectors per lane, 2 column chunks
    (500, 1030, 1, 700, 500),        # scalar columns, 5 column chunks
])
def test_embedding_forward_backward(dev, V, D, B, T, vocab_arg):
    note(f"embedding V={V} D={D} B={B} T={T} vocab_arg={vocab_arg}")
    wte, wpe, ids, g = emb_inputs(V, D, B, T, 20262 + D)
    BT = B * T
    Wte, Wpe, Ids, G = dev_t(wte), dev_t(wpe), dev_t(ids), dev_t(g)

    out = torch.empty(BT, D, device=dev)
    M.embedding_pos_forward(Wte, Wpe, Ids, out, B, T, D, vocab_arg)
    ref = O.pos_embedding_forward(wpe, O.embedding_forward(wte, ids), B, T)
    assert_exact("fused wte[id]+wpe[t]", host(out), ref)

    out2 = torch.empty(BT, D, device=dev)
    M.embedding_forward(Wte, Ids, out2, BT, D, vocab_arg)
    M.pos_embedding_forward(Wpe, out2, B, T, D)
    assert_exact("two-pass == fused", host(out2), host(out))

    r = np.random.default_rng(5)
    dwte0 = np.zeros((V, D), np.float32)
    dwte0[::3] = r.standard_normal((len(range(0, V, 3)), D), dtype=np.float32)
    dwpe0 = r.standard_normal((T, D), dtype=np.float32)
    Dwte, Dwpe = dev_t(dwte0), dev_t(dwpe0)
    M.embedding_backward(G, Ids, Dwte, BT, D, vocab_arg)
    M.pos_embedding_backward(G, Dwpe, B, T, D)
    assert_exact("dwte", host(Dwte), O.embedding_backward(g, ids, dwte0))
    assert_exact("dwpe", host(Dwpe), O.pos_embedding_backward(g, dwpe0, B, T))

    # fused token + position backward: bit-identical to the two calls
    Fwte, Fwpe = dev_t(dwte0), dev_t(dwpe0)
    M.embedding_pos_backward(G, Ids, Fwte, Fwpe, B, T, D, vocab_arg)
    assert_exact("fused dwte", host(Fwte), host(Dwte))
    assert_exact("fused dwpe", host(Fwpe), host(Dwpe))


def test_heavy_hitter_and_invalid_ids(dev):
    V, D, B, T = 300, 64, 4, 1100
    wte, wpe, ids, g = emb_inputs(V, D, B, T, 9)
    ids[: 3000] = 17            # one id repeated 3000 times: runs of 64+ entries and
                                # more list entries than one LDS window holds
    ids[3000:3010] = -5          # invalid ids: skipped by the bounded entry points
    ids[3010:3020] = V + 4
    BT = B * T
    valid = (ids >= 0) & (ids < V)
    Ids, G = dev_t(ids), dev_t(g)

    Dwte = torch.zeros(V, D, device=dev)
    M.embedding_backward(G, Ids, Dwte, BT, D, V)
    expect = O.embedding_backward(g[valid], ids[valid], np.zeros((V, D), np.float32))
    assert_exact("dwte heavy hitter", host(Dwte), expect)
    Fwte, Fwpe = torch.zeros(V, D, device=dev), torch.zeros(T, D, device=dev)
    M.embedding_pos_backward(G, Ids, Fwte, Fwpe, B, T, D, V)
    assert_exact("fused dwte heavy hitter", host(Fwte), expect)
    assert_exact("fused dwpe, every row counted", host(Fwpe),
                 O.pos_embedding_backward(g, np.zeros((T, D), np.float32), B, T))

    out = torch.empty(BT, D, device=dev)
    M.embedding_forward(dev_t(wte), Ids, out, BT, D, V)
    o = host(out)
    assert np.all(o[~valid] == 0)
    assert_exact("valid rows", o[valid], wte[ids[valid]])


def test_single_id_across_passes_and_windows(dev):
    # 40000 tokens of one id: one owning workgroup sees 3 passes over the ids
    # and 2048-entry windows in each, so the row is carried from window to
    # window and pass to pass by different waves (ordered by the barriers)
    V, D, BT = 7, 64, 40000
    r = np.random.default_rng(77)
    ids = np.full(BT, 5, np.int32)
    ids[::997] = 2                  # a second, sparse id in the same windows
    g = r.standard_normal((BT, D), dtype=np.float32)
    dwte0 = r.standard_normal((V, D), dtype=np.float32)
    Dwte = dev_t(dwte0)
    M.embedding_backward(dev_t(g), dev_t(ids), Dwte, BT, D, V)
    assert_exact("dwte single id", host(Dwte), O.embedding_backward(g, ids, dwte0))
    # fused with the position gradient, B = 8 rows of T = 5000 positions: the
    # first pass requests position loads across its scan, two more passes follow
    B, T = 8, BT // 8
    dwpe0 = r.standard_normal((T, D), dtype=np.float32)
    Fwte, Fwpe = dev_t(dwte0), dev_t(dwpe0)
    M.embedding_pos_backward(dev_t(g), dev_t(ids), Fwte, Fwpe, B, T, D, V)
    assert_exact("fused dwte single id", host(Fwte), host(Dwte))
    assert_exact("fused dwpe", host(Fwpe), O.pos_embedding_backward(g, dwpe0, B, T))


def test_trusted_ids_skip_negative(dev):
    # vocab <= 0 trusts the ids; negative ids are still skipped
    V, D, BT = 50, 32, 3000
    r = np.random.default_rng(78)
    ids = r.integers(0, V, BT).astype(np.int32)
    ids[::7] = -1
    g = r.standard_normal((BT, D), dtype=np.float32)
    Dwte = torch.zeros(V, D, device=dev)
    M.embedding_backward(dev_t(g), dev_t(ids), Dwte, BT, D, 0)
    ok = ids >= 0
    assert_exact("dwte trusted ids", host(Dwte),
                 O.embedding_backward(g[ok], ids[ok], np.zeros((V, D), np.float32)))


def test_embedding_backward_deterministic(dev):
    V, D, B, T = 50257, 768, 16, 1024
    _, _, ids, g = emb_inputs(V, D, B, T, 31)
    Ids, G = dev_t(ids), dev_t(g)
    first = None
    for _ in range(2):
        Dwte = torch.zeros(V, D, device=dev)
        M.embedding_backward(G, Ids, Dwte, B * T, D, V)
        h = host(Dwte)
        if first is None:
            first = h
        else:
            assert_exact("repeat", h, first)
    # the fused token + position backward: the same bits, call after call
    pos_first = None
    for _ in range(2):
        Fwte, Fwpe = torch.zeros(V, D, device=dev), torch.zeros(T, D, device=dev)
        M.embedding_pos_backward(G, Ids, Fwte, Fwpe, B, T, D, V)
        assert_exact("fused repeat dwte", host(Fwte), first)
        if pos_first is None:
            pos_first = host(Fwpe)
        else:
            assert_exact("fused repeat dwpe", host(Fwpe), pos_first)
    # size-independent checks: total gradient mass is preserved per column
    # and untouched rows stay zero
    touched = np.zeros(V, bool)
    touched[ids] = True
    assert np.all(first[~touched] == 0)
    np.testing.assert_allclose(first.astype(np.float64).sum(axis=0),
                               g.astype(np.float64).sum(axis=0), rtol=1e-4, atol=1e-2)


def _offset_dev(a, offset):
    """Copy to the GPU starting `offset` elements into the allocation, so an
    offset of 1 leaves the tensor 4-byte but not 16-byte aligned."""
    flat = np.ascontiguousarray(a).reshape(-1)
    buf = torch.empty(flat.size + offset, dtype=torch.from_numpy(flat[:1]).dtype, device="cuda:0")
    view = buf[offset:]
    view.copy_(torch.from_numpy(flat))
    return view


@pytest.mark.parametrize("V,D,B,T,id_off,g_off", [
    (50257, 768, 16, 1024, 1, 0),   # config 2 with 4-byte aligned ids: every id a 4-byte load
    (300, 64, 4, 1100, 1, 1),       # ids and gradient rows both off 16 bytes (scalar columns)
    (1000, 128, 3, 333, 3, 0),      # ids 12 bytes in, ragged last id group
    (17, 32, 1, 3, 1, 0),           # three tokens: fewer ids than one 16-byte load
    (5, 16, 2, 1, 0, 1),            # two tokens, one position
])
def test_embedding_backward_unaligned_ids_and_rows(dev, V, D, B, T, id_off, g_off):
    note(f"embedding unaligned V={V} D={D} B={B} T={T} id_off={id_off} g_off={g_off}")
    _, _, ids, g = emb_inputs(V, D, B, T, 4242 + T)
    ids[::5] = ids[0]              # repeated ids: runs longer than one entry
    BT = B * T
    r = np.random.default_rng(6)
    dwte0 = r.standard_normal((V, D), dtype=np.float32)
    dwpe0 = r.standard_normal((T, D), dtype=np.float32)
    Ids, G = _offset_dev(ids, id_off), _offset_dev(g, g_off)
    Dwte, Dwpe = dev_t(dwte0), dev_t(dwpe0)
    M.embedding_pos_backward(G, Ids, Dwte, Dwpe, B, T, D, V)
    assert_exact("fused dwte, unaligned", host(Dwte), O.embedding_backward(g, ids, dwte0))
    assert_exact("fused dwpe, unaligned", host(Dwpe), O.pos_embedding_backward(g, dwpe0, B, T))
    Twte = dev_t(dwte0)
    M.embedding_backward(G, Ids, Twte, BT, D, V)
    assert_exact("token dwte, unaligned", host(Twte), O.embedding_backward(g, ids, dwte0))
