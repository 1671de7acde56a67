"""BASELINE workloads on the GPU: seeded synthetic inputs in HBM, the
per-step call sequence through the C ABI, and the algorithmic byte counts
the throughput figures use.

Algorithmic bytes: every tensor a call reads is counted once and every
tensor it writes once (fp32 = 4 B, ids = 4 B); a tensor updated in place
(`+=` on a full activation, e.g. grad_residual) counts twice.  The two-pass
partial rows of the column reductions are implementation overhead and are
not counted.  Parameter-sized terms are included and negligible.
"""
from __future__ import annotations

import torch

from . import (adam_update, bias_gelu_forward, bind, gelu_backward_with_bias_backward,
               layernorm_backward_residual, layernorm_forward_save,
               residual_layernorm_forward_save)

F32 = 4


def ln_fwd_bytes(R, C):
    return F32 * (2 * R * C + 2 * R + 2 * C)


def ln_bwd_bytes(R, C):
    return F32 * (3 * R * C + 2 * R + 3 * C)


def res_ln_fwd_bytes(R, C):
    return F32 * (4 * R * C + 2 * R + 2 * C)


def ln_bwd_residual_bytes(R, C):
    return F32 * (4 * R * C + 2 * R + 3 * C)


def gelu_fwd_bytes(R, F):
    return F32 * (2 * R * F + F)


def gelu_bwd_bytes(R, F):
    return F32 * (3 * R * F + 2 * F)


def headline_bytes(R=8192, C=768, F=3072):
    return {"ln_fwd": ln_fwd_bytes(R, C), "ln_bwd": ln_bwd_bytes(R, C),
            "gelu_fwd": gelu_fwd_bytes(R, F), "gelu_bwd": gelu_bwd_bytes(R, F)}


def _randn(shape, gen, scale=1.0, shift=0.0):
    t = torch.randn(shape, device="cuda", generator=gen, dtype=torch.float32)
    if scale != 1.0:
        t.mul_(scale)
    if shift != 0.0:
        t.add_(shift)
    return t


def _sets_for(set_bytes, min_sets=2, target=1.2e9, max_sets=32):
    """Number of buffer sets so that about `target` bytes of other data pass
    between two uses of the same set (more than the 256 MB last-level cache)."""
    n = int(-(-target // max(set_bytes, 1)))
    return max(min_sets, min(max_sets, n))


class FwdBwd:
    """LayerNorm fwd+bwd on [R, C] and/or bias+GELU fwd+bwd on [R, F].

    The BASELINE headline metric is FwdBwd(8192, 768, 3072) (B=8, T=1024,
    C=768, F=4C); config 0 is the LayerNorm half at R=4096, config 1 the GELU
    half, config 4's wide sweep the LayerNorm half at [32768, 4096].

    Independent buffer sets rotate.  Step k runs the forward operations on
    set k and the backward operations on set k-1, whose forward ran one step
    earlier (as in training, where a layer's backward comes long after its
    forward).  Enough sets are used that ~1.2 GB of other data streams
    between two reads of any input, more than the 256 MB last-level cache,
    so every operation reads its inputs from HBM."""

    def __init__(self, R=8192, C=768, F=3072, ln=True, gelu=True, sets=None, seed=20260):
        self.R, self.C, self.F = R, C, F
        self.ln, self.gelu = ln, gelu
        self.seed = seed
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.bytes = {}
        if ln:
            self.bytes["ln_fwd"] = ln_fwd_bytes(R, C)
            self.bytes["ln_bwd"] = ln_bwd_bytes(R, C)
            self.gamma = _randn((C,), g, 0.02, 1.0)
            self.beta = _randn((C,), g, 0.02)
            self.dgamma = torch.zeros(C, device="cuda")
            self.dbeta = torch.zeros(C, device="cuda")
        if gelu:
            self.bytes["gelu_fwd"] = gelu_fwd_bytes(R, F)
            self.bytes["gelu_bwd"] = gelu_bwd_bytes(R, F)
            self.bias = _randn((F,), g, 0.02)
            self.dbias = torch.zeros(F, device="cuda")
        set_bytes = F32 * R * ((4 * C if ln else 0) + (4 * F if gelu else 0))
        n = sets if sets is not None else _sets_for(set_bytes, min_sets=4)
        self.sets = []
        for _ in range(n):
            s = {}
            if ln:
                s.update(x=_randn((R, C), g), dy=_randn((R, C), g),
                         y=torch.empty(R, C, device="cuda"), dx=torch.empty(R, C, device="cuda"),
                         mean=torch.empty(R, device="cuda"), rstd=torch.empty(R, device="cuda"))
            if gelu:
                s.update(h=_randn((R, F), g, 1.5), dh=_randn((R, F), g),
                         o=torch.empty(R, F, device="cuda"), gin=torch.empty(R, F, device="cuda"))
            self.sets.append(s)
        self.step_bytes = sum(self.bytes.values())
        self._bound = {}
        if ln:
            for s in self.sets:  # every set's saved statistics exist before its backward
                layernorm_forward_save(s["x"], self.gamma, self.beta, s["y"], s["mean"],
                                       s["rstd"], R, C, 1e-5)

    def ops(self, k):
        """The step's calls as (name, callable) pairs, bound once per buffer
        set (C-ABI calls with their arguments already converted, so the host
        issues a step in a few microseconds)."""
        n = len(self.sets)
        key = k % n
        if key not in self._bound:
            f = self.sets[key]
            b = self.sets[(k - 1) % n]
            R, C, F = self.R, self.C, self.F
            out = []
            if self.ln:
                out.append(("ln_fwd", bind("mi_layernorm_forward_save", f["x"], self.gamma,
                                           self.beta, f["y"], f["mean"], f["rstd"], R, C, 1e-5)))
            if self.gelu:
                out.append(("gelu_fwd", bind("mi_bias_gelu_forward", f["h"], self.bias, f["o"],
                                             R, F)))
            if self.ln:
                out.append(("ln_bwd", bind("mi_layernorm_backward", b["dy"], b["x"], b["mean"],
                                           b["rstd"], self.gamma, b["dx"], self.dgamma,
                                           self.dbeta, R, C)))
            if self.gelu:
                out.append(("gelu_bwd", bind("mi_gelu_backward_with_bias_backward", b["h"],
                                             self.bias, b["dh"], b["gin"], self.dbias, R, F)))
            self._bound[key] = out
        return self._bound[key]

    def step(self, k):
        for _, fn in self.ops(k):
            fn()

    def host_inputs(self, k=0):
        s = self.sets[k % len(self.sets)]
        d = {n: t.cpu().numpy() for n, t in s.items()
             if n in ("x", "dy", "h", "dh")}
        if self.ln:
            d.update(gamma=self.gamma.cpu().numpy(), beta=self.beta.cpu().numpy())
        if self.gelu:
            d.update(bias=self.bias.cpu().numpy())
        return d


def Headline(sets=None):
    """The BASELINE metric's workload."""
    return FwdBwd(8192, 768, 3072, sets=sets)


class BlockSequence:
    """One GPT-2 block's non-GEMM sequence repeated over `layers` layers
    (BASELINE configs 3 and 4).  Per layer, forward: r1 = r + a (fused with
    LN1), r2 = r1 + m (fused with LN2), bias+GELU on [R, F]; backward in
    reverse: GELU bwd + dbias, LN2 bwd accumulated into the residual-stream
    gradient, LN1 bwd likewise.  a, m, the GELU pre-activation and the
    upstream gradients stand in for the GEMM outputs (synthetic N(0,1))."""

    def __init__(self, R, C, F, layers, seed=20263, shared_inputs=False):
        self.R, self.C, self.F, self.L = R, C, F, layers
        self.seed = seed
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        n_in = 1 if shared_inputs else layers
        self.inp = [{"a": _randn((R, C), g), "m": _randn((R, C), g), "h": _randn((R, F), g),
                     "gy1": _randn((R, C), g), "gy2": _randn((R, C), g), "gh": _randn((R, F), g)}
                    for _ in range(n_in)]
        self.params = [{"g1": _randn((C,), g, 0.02, 1.0), "b1": _randn((C,), g, 0.02),
                        "g2": _randn((C,), g, 0.02, 1.0), "b2": _randn((C,), g, 0.02),
                        "bias": _randn((F,), g, 0.02)} for _ in range(layers)]
        self.grads = [{k: torch.zeros_like(v) for k, v in p.items()} for p in self.params]
        self.r0 = _randn((R, C), g)
        self.act = [{"r1": torch.empty(R, C, device="cuda"), "r2": torch.empty(R, C, device="cuda"),
                     "y1": torch.empty(R, C, device="cuda"), "y2": torch.empty(R, C, device="cuda"),
                     "m1": torch.empty(R, device="cuda"), "s1": torch.empty(R, device="cuda"),
                     "m2": torch.empty(R, device="cuda"), "s2": torch.empty(R, device="cuda"),
                     "o": torch.empty(R, F, device="cuda"), "gin": torch.empty(R, F, device="cuda")}
                    for _ in range(layers)]
        self.gres = torch.empty(R, C, device="cuda")
        self.step_bytes = layers * (2 * res_ln_fwd_bytes(R, C) + gelu_fwd_bytes(R, F)
                                    + gelu_bwd_bytes(R, F) + 2 * ln_bwd_residual_bytes(R, C))

    def _in(self, l):
        return self.inp[l % len(self.inp)]

    def step(self, k):
        """One training step's non-GEMM work: forward over all layers, then
        backward over all layers, issued as bound C-ABI calls.

        The residual-stream gradient buffer is set to a synthetic upstream
        gradient once, before the first step; every step's backward then
        accumulates its 2 L LayerNorm-backward terms onto the value it finds
        (`+=`, as the reference's layernorm_backward_residual does).  In the
        reference that buffer is written by the output-projection GEMM at the
        start of each backward (FINAL_CLEAN_CODE/src/model/transformer.cu:459,
        gemm_tiled_BT into act.grad_residual2), which is outside this path,
        so no stand-in for it runs inside the step: the kernels, their
        arguments and the bytes they move are the same every step."""
        if not hasattr(self, "_calls"):
            g = torch.Generator(device="cuda")
            g.manual_seed(11)
            self.gtop = _randn((self.R, self.C), g)
            self.gres.copy_(self.gtop)
            self._calls = self._bind_step()
        for fn in self._calls:
            fn()

    def _bind_step(self):
        R, C, F = self.R, self.C, self.F
        calls = []
        r = self.r0
        for l in range(self.L):
            i, p, a = self._in(l), self.params[l], self.act[l]
            calls.append(bind("mi_residual_layernorm_forward_save", r, i["a"], p["g1"], p["b1"],
                              a["r1"], a["y1"], a["m1"], a["s1"], R, C, 1e-5))
            calls.append(bind("mi_residual_layernorm_forward_save", a["r1"], i["m"], p["g2"],
                              p["b2"], a["r2"], a["y2"], a["m2"], a["s2"], R, C, 1e-5))
            calls.append(bind("mi_bias_gelu_forward", i["h"], p["bias"], a["o"], R, F))
            r = a["r2"]
        for l in reversed(range(self.L)):
            i, p, a, gr = self._in(l), self.params[l], self.act[l], self.grads[l]
            calls.append(bind("mi_gelu_backward_with_bias_backward", i["h"], p["bias"], i["gh"],
                              a["gin"], gr["bias"], R, F))
            # LN2 normalised r2 = r1 + m and LN1 normalised r1 = r + a; the
            # residual adds pass the stream gradient through unchanged.
            calls.append(bind("mi_layernorm_backward_residual", i["gy2"], a["r2"], a["m2"],
                              a["s2"], p["g2"], self.gres, gr["g2"], gr["b2"], R, C))
            calls.append(bind("mi_layernorm_backward_residual", i["gy1"], a["r1"], a["m1"],
                              a["s1"], p["g1"], self.gres, gr["g1"], gr["b1"], R, C))
        return calls

    def forward(self):
        R, C, F = self.R, self.C, self.F
        r = self.r0
        for l in range(self.L):
            i, p, a = self._in(l), self.params[l], self.act[l]
            residual_layernorm_forward_save(r, i["a"], p["g1"], p["b1"], a["r1"], a["y1"], a["m1"],
                                            a["s1"], R, C, 1e-5)
            residual_layernorm_forward_save(a["r1"], i["m"], p["g2"], p["b2"], a["r2"], a["y2"],
                                            a["m2"], a["s2"], R, C, 1e-5)
            bias_gelu_forward(i["h"], p["bias"], a["o"], R, F)
            r = a["r2"]
        return r

    def backward(self, gres_init):
        R, C, F = self.R, self.C, self.F
        self.gres.copy_(gres_init)
        for l in reversed(range(self.L)):
            i, p, a, gr = self._in(l), self.params[l], self.act[l], self.grads[l]
            gelu_backward_with_bias_backward(i["h"], p["bias"], i["gh"], a["gin"], gr["bias"], R, F)
            layernorm_backward_residual(i["gy2"], a["r2"], a["m2"], a["s2"], p["g2"], self.gres,
                                        gr["g2"], gr["b2"], R, C)
            layernorm_backward_residual(i["gy1"], a["r1"], a["m1"], a["s1"], p["g1"], self.gres,
                                        gr["g1"], gr["b1"], R, C)
        return self.gres


class Embedding:
    """ids U[0, V) for B x T, wte [V, D], wpe [T, D].
    `sets` independent id / gradient / output sets rotate between steps."""

    def __init__(self, V=50257, D=768, B=16, T=1024, sets=4, seed=20262):
        self.V, self.D, self.B, self.T = V, D, B, T
        self.seed = seed
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.wte = _randn((V, D), g, 0.02)
        self.wpe = _randn((T, D), g, 0.02)
        self.dwte = torch.zeros(V, D, device="cuda")
        self.dwpe = torch.zeros(T, D, device="cuda")
        BT = B * T
        self.sets = []
        for _ in range(sets):
            ids = torch.randint(0, V, (BT,), device="cuda", generator=g, dtype=torch.int32)
            self.sets.append({"ids": ids, "dout": _randn((BT, D), g),
                              "out": torch.empty(BT, D, device="cuda"),
                              "distinct": int(torch.unique(ids).numel())})
        self.distinct = sum(s["distinct"] for s in self.sets) / len(self.sets)
        self.fwd_bytes = F32 * (BT + 2 * BT * D + T * D)
        self.bwd_bytes = int(F32 * (BT * D + BT + 2 * self.distinct * D + 2 * T * D))
        self.bytes = {"emb_fwd": self.fwd_bytes, "emb_bwd": self.bwd_bytes}
        self.step_bytes = self.fwd_bytes + self.bwd_bytes
        self._bound = {}

    def ops(self, k):
        key = k % len(self.sets)
        if key not in self._bound:
            s = self.sets[key]
            B, T, D, V = self.B, self.T, self.D, self.V
            self._bound[key] = [
                ("emb_fwd", bind("mi_embedding_pos_forward", self.wte, self.wpe, s["ids"], s["out"],
                                 B, T, D, V)),
                ("emb_bwd", bind("mi_embedding_pos_backward", s["dout"], s["ids"], self.dwte,
                                 self.dwpe, B, T, D, V)),
            ]
        return self._bound[key]

    def step(self, k):
        for _, fn in self.ops(k):
            fn()


class CrossEntropy:
    """Softmax cross-entropy of the reference model's loss
    (FINAL_CLEAN_CODE/src/model/transformer.cu:402-407,
    cross_entropy_forward_v2): logits [B*T, V] ~ N(0, 2^2), targets U[0, V).
    Algorithmic bytes: logits read, gradient written, targets read, losses
    written, 4(2 R V + 2 R).  `sets` logits / gradient pairs rotate."""

    def __init__(self, R=8192, V=50257, sets=2, seed=20268):
        self.R, self.V = R, V
        self.seed = seed
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.sets = []
        for _ in range(sets):
            self.sets.append({
                "logits": _randn((R, V), g, 2.0),
                "targets": torch.randint(0, V, (R,), device="cuda", generator=g,
                                         dtype=torch.int32),
                "grad": torch.empty(R, V, device="cuda"),
                "losses": torch.empty(R, device="cuda"),
                "loss": torch.empty(1, device="cuda")})
        self.step_bytes = F32 * (2 * R * V + 2 * R)
        self.bytes = {"cross_entropy": self.step_bytes}
        self._bound = {}

    def ops(self, k):
        key = k % len(self.sets)
        if key not in self._bound:
            s = self.sets[key]
            self._bound[key] = [("cross_entropy", bind(
                "mi_cross_entropy_forward_v2", s["logits"], s["targets"], s["grad"], s["losses"],
                s["loss"], self.R, self.V))]
        return self._bound[key]

    def step(self, k):
        for _, fn in self.ops(k):
            fn()


class AdamStep:
    """The reference's optimizer step, TransformerModel::update_adam
    (FINAL_CLEAN_CODE/src/model/transformer.cu:619-636), over a flat buffer
    of GPT-2 small's parameter count: gradient norm², clip scale, clipped
    Adam.  Algorithmic bytes 4 n (norm² read) + 28 n (Adam: param, grad, m, v
    read; param, m, v written) = 32 n."""

    def __init__(self, n=124_439_808, seed=20269):
        self.n = n
        self.seed = seed
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.param = _randn((n,), g, 0.02)
        self.grad = _randn((n,), g, 1e-3)
        self.m = torch.zeros(n, device="cuda")
        self.v = torch.zeros(n, device="cuda")
        self.norm_sq = torch.empty(1, device="cuda")
        self.clip = torch.empty(1, device="cuda")
        self.step_bytes = 32 * n
        self.bytes = {"adam_update": self.step_bytes}

    def ops(self, k):
        return [("adam_update", lambda: adam_update(self.param, self.grad, self.m, self.v, self.n,
                                                    3e-4, 0.9, 0.999, 1e-8, k + 1, 1.0,
                                                    self.norm_sq, self.clip))]

    def step(self, k):
        for _, fn in self.ops(k):
            fn()


class Relu16:
    """The reference's fp16 activation-storage path at config 1's shape
    (FINAL_CLEAN_CODE/src/kernels/activations.cu:199-217,285-323):
    bias_relu_forward_to_half (fp32 in, fp16 out) and
    relu_backward_with_bias_backward_half_mask (fp16 mask, fp32 grads) on
    [8192, 3072].  Bytes: fwd 4N + 2N + 4F, bwd 2N + 4N + 4N + 8F."""

    def __init__(self, R=8192, F=3072, sets=4, seed=20270):
        self.R, self.F = R, F
        self.seed = seed
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.bias = _randn((F,), g, 0.02)
        self.dbias = torch.zeros(F, device="cuda")
        self.sets = [{"h": _randn((R, F), g, 1.5), "dh": _randn((R, F), g),
                      "o16": torch.empty(R, F, dtype=torch.float16, device="cuda"),
                      "gin": torch.empty(R, F, device="cuda")} for _ in range(sets)]
        N = R * F
        self.bytes = {"relu16_fwd": 6 * N + F32 * F, "relu16_bwd": 10 * N + 8 * F}
        self.step_bytes = sum(self.bytes.values())
        self._bound = {}

    def ops(self, k):
        key = k % len(self.sets)
        if key not in self._bound:
            s, p = self.sets[key], self.sets[(k - 1) % len(self.sets)]
            R, F = self.R, self.F
            self._bound[key] = [
                ("relu16_fwd", bind("mi_bias_relu_forward_to_half", s["h"], self.bias, s["o16"],
                                    R, F)),
                ("relu16_bwd", bind("mi_relu_backward_with_bias_backward_half_mask", p["o16"],
                                    p["dh"], p["gin"], self.dbias, R, F))]
        return self._bound[key]

    def step(self, k):
        for _, fn in self.ops(k):
            fn()


class RefShapes:
    """The reference's own kernel benchmarks, at its own shapes and with its
    own loops, run in C++ through include/kernels.h (bench/refshapes.cpp,
    built as refshapes_bench next to the library), as the reference's are:
    from Python the ctypes call overhead (~7 us) would exceed these kernels.
    The same call repeats on the same buffers, so the tensors stay
    cache-resident, as in the reference.

      * fused-versus-unfused pairs of FINAL_CLEAN_CODE/tests/
        test_fusion_benchmark.cu (bias+ReLU 2048x512; residual+LN forward and
        LN backward+residual 2048x128) and the LN forward of
        results/correctness_matrix_85267.md:24 (2048x128).  Bytes follow the
        reference's model (profile_fusion_kernels.cu:30-55): a multiple of
        nbytes = rows*cols*4 per call; the LN forward uses the "effective BW"
        2*rows*cols*4 of correctness_matrix.  Reference figures on its Quadro
        RTX 6000 (672 GB/s): CUDA-event time per call
        (results/final_clean_main_table.csv:57-65; correctness_matrix_85267.md:24
        for the LN forward) and Nsight Compute kernel time
        (results/roofline_fusion.csv:2-7).
      * the LayerNorm bandwidth grid of tests/benchmark_all.cu:124-163 (six
        shapes, bytes 2*rows*cols*4 as it counts them), with its logged
        event times (FINAL_CLEAN_CODE_/logs/full_validation_88905.out:209-214,
        and the slower run full_validation_89398.out:214-219);
      * the LayerNorm forward of tests/deep_profile.cu:121-173 at
        2048x{128,256,512} (bytes (2*rows*cols + 2*cols)*4 as it counts
        them); the reference tree holds no logged output of it.

    Context, not a same-node comparison."""

    CASES = {
        # name: (rows, cols, bytes in units of nbytes, ref event us, ref ncu us)
        "ln_fwd": (2048, 128, 2.0, 7.0, None),
        "residual_ln_unfused": (2048, 128, 9.0, 9.9, 16.80),
        "residual_ln_fused": (2048, 128, 8.0, 7.5, 11.04),
        "ln_bwd_residual_unfused": (2048, 128, 12.0, 22.2, 34.02),
        "ln_bwd_residual_fused": (2048, 128, 10.0, 20.0, 28.99),
        "bias_relu_unfused": (2048, 512, 5.0, 22.6, 32.90),
        "bias_relu_fused": (2048, 512, 4.0, 15.7, 14.62),
    }
    # benchmark_all.cu's grid: (rows, cols) -> (ref event us, slower run us)
    GRID = {(1024, 64): (3.3, 4.5), (1024, 128): (4.5, 6.1), (2048, 128): (7.0, 9.4),
            (4096, 128): (11.6, 15.5), (2048, 256): (11.7, 15.7), (2048, 512): (21.5, 25.1)}
    DEEP = [(2048, 128), (2048, 256), (2048, 512)]
    HARNESS = "refshapes_bench"

    def __init__(self):
        import os
        self.seed = 42
        self.bytes = {k: int(m * r * c * F32) for k, (r, c, m, _, _) in self.CASES.items()}
        for (r, c) in self.GRID:
            self.bytes[f"ln_grid_{r}x{c}"] = 2 * r * c * F32
        for (r, c) in self.DEEP:
            self.bytes[f"ln_deep_{r}x{c}"] = (2 * r * c + 2 * c) * F32
        self.step_bytes = sum(self.bytes.values())
        self.harness = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    self.HARNESS)

    def names(self):
        return list(self.bytes)

    def published(self, name):
        """The reference's figures for a case (None where it has none)."""
        if name in self.CASES:
            _, _, _, ev, ncu = self.CASES[name]
            return {"event_us": ev, "ncu_us": ncu}
        if name.startswith("ln_grid_"):
            r, c = (int(v) for v in name[len("ln_grid_"):].split("x"))
            ev, ev2 = self.GRID[(r, c)]
            return {"event_us": ev, "event_us_other_run": ev2, "ncu_us": None}
        return {"event_us": None, "ncu_us": None}

    def run(self, scale=1):
        """Runs the C++ harness; returns {case: {"us": per call, "calls": timed calls}}."""
        import json
        import subprocess
        out = subprocess.run([self.harness, str(scale)], capture_output=True, text=True,
                             check=True, timeout=300).stdout
        return json.loads(out.strip().splitlines()[-1])
