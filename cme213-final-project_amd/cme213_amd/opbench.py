"""Runs each operation of the headline step (and a copy kernel of known size)
a few times with the last-level cache flushed before each call, for
rocprofv3 counter collection, e.g.

  rocprofv3 --pmc FETCH_SIZE -d OUT -o pmc -- \
      python3 cme213-final-project_amd/cme213_amd/opbench.py

The copy kernel (relu_forward over [8192, 3072]: 96 MiB read, 96 MiB
written) calibrates what the counters read for a known number of bytes.
--set others runs the embedding, cross-entropy and optimizer calls instead.
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import torch  # noqa: E402

import cme213_amd as M  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=3)
    ap.add_argument("--set", choices=("headline", "others"), default="headline",
                    help="headline: the four operations of the headline step and the copy "
                         "kernel; others: the embedding forward/backward (config 2), the "
                         "softmax cross-entropy and the optimizer step")
    args = ap.parse_args()
    if args.set == "others":
        return others(args.iters)
    R, C, F = 8192, 768, 3072
    g = torch.Generator(device="cuda")
    g.manual_seed(3)

    def rn(*s):
        return torch.randn(*s, device="cuda", generator=g)

    x, dy = rn(R, C), rn(R, C)
    y, dx = torch.empty(R, C, device="cuda"), torch.empty(R, C, device="cuda")
    m, s = torch.empty(R, device="cuda"), torch.empty(R, device="cuda")
    h, dh = rn(R, F), rn(R, F)
    o, gin = torch.empty(R, F, device="cuda"), torch.empty(R, F, device="cuda")
    gm, bt, bias = rn(C) * 0.02 + 1, rn(C) * 0.02, rn(F) * 0.02
    dg, db, dbi = (torch.zeros(C, device="cuda"), torch.zeros(C, device="cuda"),
                   torch.zeros(F, device="cuda"))
    flush_src = torch.empty(128 << 20, device="cuda")  # 512 MiB, twice the last-level cache
    flush_dst = torch.empty_like(flush_src)

    def flush():
        flush_dst.copy_(flush_src)
        torch.cuda.synchronize()

    calls = [
        ("copy relu_forward [8192,3072]", lambda: M.relu_forward(h, o, R * F)),
        ("layernorm_forward_save [8192,768]",
         lambda: M.layernorm_forward_save(x, gm, bt, y, m, s, R, C)),
        ("layernorm_backward [8192,768]",
         lambda: M.layernorm_backward(dy, x, m, s, gm, dx, dg, db, R, C)),
        ("bias_gelu_forward [8192,3072]", lambda: M.bias_gelu_forward(h, bias, o, R, F)),
        ("gelu_backward_with_bias_backward [8192,3072]",
         lambda: M.gelu_backward_with_bias_backward(h, bias, dh, gin, dbi, R, F)),
    ]
    for _ in range(args.iters):
        for name, fn in calls:
            flush()
            fn()
            torch.cuda.synchronize()
    print("opbench: ran", ", ".join(n for n, _ in calls), flush=True)


def others(iters):
    g = torch.Generator(device="cuda")
    g.manual_seed(5)

    def rn(*s, scale=1.0):
        return torch.randn(*s, device="cuda", generator=g) * scale

    V, D, B, T = 50257, 768, 16, 1024
    wte, wpe = rn(V, D, scale=0.02), rn(T, D, scale=0.02)
    ids = torch.randint(0, V, (B * T,), device="cuda", generator=g, dtype=torch.int32)
    out, dout = torch.empty(B * T, D, device="cuda"), rn(B * T, D)
    dwte, dwpe = torch.zeros(V, D, device="cuda"), torch.zeros(T, D, device="cuda")
    R, VV = 8192, 50257
    logits, tg = rn(R, VV, scale=2.0), torch.randint(0, VV, (R,), device="cuda", generator=g,
                                                     dtype=torch.int32)
    grad, losses, loss = (torch.empty(R, VV, device="cuda"), torch.empty(R, device="cuda"),
                          torch.empty(1, device="cuda"))
    n = 124_439_808
    prm, grd = rn(n, scale=0.02), rn(n, scale=1e-3)
    mm, vv = torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda")
    nsq, clip = torch.empty(1, device="cuda"), torch.empty(1, device="cuda")
    flush_src = torch.empty(128 << 20, device="cuda")
    flush_dst = torch.empty_like(flush_src)

    def flush():
        flush_dst.copy_(flush_src)
        torch.cuda.synchronize()

    calls = [
        ("embedding_pos_forward (config 2)",
         lambda: M.embedding_pos_forward(wte, wpe, ids, out, B, T, D, V)),
        ("embedding_pos_backward (config 2)",
         lambda: M.embedding_pos_backward(dout, ids, dwte, dwpe, B, T, D, V)),
        ("cross_entropy_forward_v2 [8192,50257]",
         lambda: M.cross_entropy_forward_v2(logits, tg, grad, losses, loss, R, VV)),
        ("adam_update (124,439,808 parameters)",
         lambda: M.adam_update(prm, grd, mm, vv, n, 3e-4, 0.9, 0.999, 1e-8, 1, 1.0, nsq, clip)),
    ]
    for _ in range(iters):
        for name, fn in calls:
            flush()
            fn()
            torch.cuda.synchronize()
    print("opbench: ran", ", ".join(n for n, _ in calls), flush=True)


if __name__ == "__main__":
    main()
