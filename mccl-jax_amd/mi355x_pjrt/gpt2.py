"""One-GPU training step of a GPT-2-style decoder on the mk_* kernels
(config C5: 12 layers, d_model 768, 12 heads, seq 1024, batch 8, vocab 50257,
bf16 parameters and activations, fp32 Adam).

This is the computation the reference's data-parallel loop jits on each rank
(temp/dp_train.py:67-76: value_and_grad of the loss, then the Adam update of
lines 71-75), for a pre-LayerNorm decoder with tied input/output embeddings,
GELU(tanh) MLP and causal attention, without the pmean (one GPU).  Every
operation is a call through the C-ABI of include/mk_kernels.h:

  forward   gather + position add, per layer LN -> QKV GEMM (+ bias) -> causal
            attention -> output GEMM -> residual + bias add -> LN -> FC GEMM,
            bias add -> GELU -> projection GEMM -> residual + bias add; final
            LN, logits GEMM against the embedding table, fused softmax
            cross-entropy (loss rows and the logit gradient, in place)
  backward  the transposed GEMMs (weight gradients straight to fp32), flash
            attention backward, GELU backward fused with the MLP bias column
            sums, LayerNorm backward fused with the residual add and the
            projection-bias column sums, position-embedding column sum,
            deterministic scatter-add of the token gradient into the
            embedding gradient
  update    one Adam launch over all parameters (fp32 master, m, v; bf16
            working copy rewritten), lr and bias corrections read from a
            device buffer so the whole step can be replayed as a HIP graph

The per-layer GEMMs run on the hand-written MFMA GEMM (mk_gemm; the QKV bias
in its epilogue, the other biases in the elementwise pass that follows) and
the weight gradients on its split-K form (mk_gemm_splitk).  The logits and
their gradient live in one bf16 buffer whose rows are padded from 50257 to
50264 elements (16-byte multiples), so the two gradient products through the
tied embedding take aligned operand rows on the hand-written kernels: the
embedding gradient on mk_gemm, the hidden-state gradient (a contraction over
the 50257 classes into a 8192 x 768 result) on mk_gemm_splitk_typed, 8
slices.  The logits product itself (K = 768 into 8192 x 50257) stays on
rocBLAS (mk_gemm_blas), which runs it 10-25% faster than the tiled kernel.
Every other operation is a hand-written kernel.  All parameters live in five flat buffers (fp32 master, bf16 working copy,
fp32 gradient, fp32 m, fp32 v), each parameter a 64-element-aligned slice, so
the optimizer is a single launch and every gradient is written in place.  The
step is prepared once as a list of bound calls (device pointers and shapes
fixed), so running it costs a few microseconds of host time per launch, and
the list can be captured into a HIP graph.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import kernels as K
from ._lib import load_kernels

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double

BF16, F32, S32 = K.MK["BF16"], K.MK["F32"], K.MK["S32"]


@dataclass(frozen=True)
class GPT2Config:
    n_layer: int = 12
    d_model: int = 768
    n_head: int = 12
    seq: int = 1024
    batch: int = 8
    vocab: int = 50257
    ln_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_head

    @property
    def d_ff(self) -> int:
        return 4 * self.d_model

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def param_shapes(self):
        """(name, shape) of every parameter, in buffer order."""
        d, f = self.d_model, self.d_ff
        out = [("wte", (self.vocab, d)), ("wpe", (self.seq, d))]
        for l in range(self.n_layer):
            p = f"h{l}."
            out += [(p + "ln1_g", (d,)), (p + "ln1_b", (d,)), (p + "w_qkv", (d, 3 * d)), (p + "b_qkv", (3 * d,)),
                    (p + "w_o", (d, d)), (p + "b_o", (d,)), (p + "ln2_g", (d,)), (p + "ln2_b", (d,)),
                    (p + "w_fc", (d, f)), (p + "b_fc", (f,)), (p + "w_pr", (f, d)), (p + "b_pr", (d,))]
        out += [("lnf_g", (d,)), ("lnf_b", (d,))]
        return out

    def flops_per_step(self) -> float:
        """Model FLOPs of one training step (forward + backward = 3x forward),
        counting the causal attention products at half their dense size."""
        d, T = self.d_model, self.tokens
        per_layer = 2 * T * (d * 3 * d + d * d + 2 * d * self.d_ff)
        attn = 2 * 2 * self.batch * self.n_head * self.seq * self.seq * self.head_dim / 2
        head = 2 * T * d * self.vocab
        return 3.0 * (self.n_layer * (per_layer + attn) + head)


def init_params(cfg: GPT2Config, seed: int = 0) -> dict:
    """Random-init weights (numpy fp32): N(0, 0.02) matrices and embeddings,
    LayerNorm gamma 1 / beta 0, biases 0; seeded numpy PCG64."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in cfg.param_shapes():
        leaf = name.split(".")[-1]
        if leaf.endswith("_g"):
            a = np.ones(shape, np.float32)
        elif leaf.startswith("b_") or leaf.endswith("_b"):
            a = np.zeros(shape, np.float32)
        else:
            a = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        out[name] = a
    return out


class _Call:
    """A C-ABI call with its arguments converted once."""

    __slots__ = ("fn", "args", "name")

    def __init__(self, fn, args, name):
        self.fn, self.args, self.name = fn, tuple(args), name

    def __call__(self):
        rc = self.fn(*self.args)
        if rc != 0:
            K._check(rc, self.name)


class GPT2TrainStep:
    """Buffers, parameters and the prepared launch list of one training step."""

    # K-slices of the fp32 weight-gradient GEMMs (dW = Xᵀ dY, K = tokens):
    # their few output tiles leave most CUs idle unless K is split.  Counts
    # measured at C5 on one MI355X (mk_gemm_splitk with 1, 2, 4, 8 and 16
    # slices; TFLOP/s dw_o 102/179/281/294/260, dw_qkv 304/493/596/462/315,
    # dw_fc and dw_pr 415/593/621/514/367).
    DW_SPLITS = {"dw_o": 8, "dw_qkv": 4, "dw_fc": 4, "dw_pr": 4}
    # the MLP's GELU forward / backward in the epilogues of its products
    # (mk_gemm_bias_gelu / mk_gemm_gelu_bwd) rather than separate passes.
    # Same-process A/B of the step (ms): separate 12.94, forward fused 12.86,
    # both 12.92, backward only 13.00 -- the backward's epilogue (reading the
    # pre-activations, the column pass) costs more than the pass it replaces
    FUSE_GELU_FWD = True
    FUSE_GELU_BWD = False
    # the hidden-state gradient through the embedding (K = vocabulary): bf16
    # out, split along K in uneven slices (measured: 8 slices 664 us, 2 693,
    # unsplit 910; rocBLAS 682-687)
    DHF_SPLITS = 8
    # products on the library GEMM (measured faster there; see the module doc)
    BLAS_GEMMS = ("logits",)

    def __init__(self, cfg: GPT2Config, params: dict | None = None, seed: int = 0, lr: float = 3e-4,
                 b1: float = 0.9, b2: float = 0.999, adam_eps: float = 1e-8, device="cuda", stream=None):
        if cfg.head_dim not in (64, 128):
            raise ValueError("head_dim must be 64 or 128 (mk_sdpa_fwd)")
        if cfg.d_model > 2048 or cfg.d_model % 8:
            raise ValueError("d_model must be a multiple of 8, at most 2048 (mk_layernorm_bwd)")
        self.cfg, self.dev = cfg, torch.device(device)
        self.lr, self.b1, self.b2, self.adam_eps = lr, b1, b2, adam_eps
        self.t = 0  # Adam step count
        self.stream = torch.cuda.current_stream(self.dev) if stream is None else stream
        self.lib = load_kernels()
        # ---- parameters: one slice per parameter in five flat buffers
        self.offsets, off = {}, 0
        for name, shape in cfg.param_shapes():
            n = int(np.prod(shape))
            self.offsets[name] = (off, shape)
            off += (n + 63) // 64 * 64
        self.n_params = sum(int(np.prod(s)) for _, s in cfg.param_shapes())
        self.n_flat = off
        f32 = dict(dtype=torch.float32, device=self.dev)
        self.master = torch.zeros(off, **f32)
        self.param = torch.zeros(off, dtype=torch.bfloat16, device=self.dev)
        self.grad = torch.zeros(off, **f32)
        self.m = torch.zeros(off, **f32)
        self.v = torch.zeros(off, **f32)
        self.hyper = torch.zeros(3, **f32)  # lr, bc1, bc2 of the current step (device scalars)
        # pinned staging for those scalars: a ring, so a step's upload never
        # waits for the stream (a buffer is reused only after the copy that
        # last read it has run, four steps back)
        self._hyper_host = [torch.zeros(3, dtype=torch.float32, pin_memory=True) for _ in range(4)]
        self._hyper_done = [None] * 4
        self.graph = None
        self.load(params if params is not None else init_params(cfg, seed))
        self._alloc()
        self.ids = torch.zeros(cfg.tokens, dtype=torch.int32, device=self.dev)
        self.labels = torch.zeros(cfg.tokens, dtype=torch.int32, device=self.dev)
        self.calls = self._build()

    # ------------------------------------------------------------------ params
    def view(self, buf, name):
        off, shape = self.offsets[name]
        return buf[off:off + int(np.prod(shape))].view(shape)

    def load(self, params: dict):
        for name, (off, shape) in self.offsets.items():
            a = torch.from_numpy(np.ascontiguousarray(params[name], dtype=np.float32)).reshape(shape)
            self.view(self.master, name).copy_(a.to(self.dev))
        rc = self.lib.mk_convert(_P(self.stream.cuda_stream), F32, BF16, self.n_flat, _P(self.master.data_ptr()),
                                 _P(self.param.data_ptr()))
        K._check(rc, "mk_convert")

    def params_numpy(self, buf=None) -> dict:
        buf = self.master if buf is None else buf
        return {n: self.view(buf, n).float().cpu().numpy() for n in self.offsets}

    # ------------------------------------------------------------------ buffers
    def _alloc(self):
        c, dev = self.cfg, self.dev
        T, d, L = c.tokens, c.d_model, c.n_layer
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.x = [torch.empty(T, d, **bf) for _ in range(L + 1)]
        self.h1 = [torch.empty(T, d, **bf) for _ in range(L)]
        self.qkv = [torch.empty(T, 3 * d, **bf) for _ in range(L)]
        self.att = [torch.empty(T, d, **bf) for _ in range(L)]
        self.lse = [torch.empty(c.batch, c.n_head, c.seq, dtype=torch.float32, device=dev) for _ in range(L)]
        self.xm = [torch.empty(T, d, **bf) for _ in range(L)]
        self.h2 = [torch.empty(T, d, **bf) for _ in range(L)]
        self.f = [torch.empty(T, c.d_ff, **bf) for _ in range(L)]
        self.g = [torch.empty(T, c.d_ff, **bf) for _ in range(L)]
        self.hf = torch.empty(T, d, **bf)
        # logits, then their gradient in place, rows padded to a 16-byte
        # multiple (the padding is never written)
        self.vocab_pitch = (c.vocab + 7) // 8 * 8
        self.logits = torch.zeros(T, self.vocab_pitch, **bf)
        self.tmp = torch.empty(T, d, **bf)
        self.dx = torch.empty(T, d, **bf)
        self.dh = torch.empty(T, d, **bf)
        self.dff = torch.empty(T, c.d_ff, **bf)
        self.dqkv = torch.empty(T, 3 * d, **bf)
        self.dx32 = torch.empty(T, d, dtype=torch.float32, device=dev)
        self.loss_rows = torch.empty(T, dtype=torch.float32, device=dev)
        self.loss_sum = torch.empty(1, dtype=torch.float32, device=dev)
        lib = self.lib
        sk = [lib.mk_gemm_splitk_workspace_bytes(d, n, self.DW_SPLITS.get(t, 1))
              for t, n in (("dw_o", d), ("dw_qkv", 3 * d), ("dw_fc", c.d_ff))]
        sk.append(lib.mk_gemm_splitk_workspace_bytes(c.d_ff, d, self.DW_SPLITS.get("dw_pr", 1)))
        sk.append(lib.mk_gemm_splitk_workspace_bytes(T, d, self.DHF_SPLITS))
        ws = max(*sk, lib.mk_col_sum_workspace_bytes(T, c.d_ff), lib.mk_col_sum_workspace_bytes(c.batch, c.seq * d),
                 lib.mk_layernorm_bwd_workspace_bytes(T, d), lib.mk_gemm_gelu_bwd_workspace_bytes(T, c.d_ff),
                 lib.mk_sdpa_bwd_workspace_bytes(c.batch, c.n_head, c.seq, c.seq, c.d_model // c.n_head),
                 lib.mk_scatter_add_workspace_bytes(c.vocab, T))
        self.ws = torch.empty(int(ws), dtype=torch.uint8, device=dev)

    # ------------------------------------------------------------------ launch list
    def _build(self):
        c, lib = self.cfg, self.lib
        T, d, F, V, L = c.tokens, c.d_model, c.d_ff, c.vocab, c.n_layer
        B, H, S, hd = c.batch, c.n_head, c.seq, c.head_dim
        st = _P(self.stream.cuda_stream)
        ws = _P(self.ws.data_ptr())
        calls = []

        def P(t, off=0):
            return _P(t.data_ptr() + off * t.element_size())

        def W(name):
            return P(self.view(self.param, name))

        def G(name):
            return P(self.view(self.grad, name))

        def gemm(ab, ct, M, N, Kd, a, a_ms, a_ks, b, b_ks, b_ns, cptr, c_ms, tag="gemm", bias=None):
            # hand-written GEMM (optionally + bias); the fp32 weight gradients
            # (few output tiles, K = tokens) split along K; the vocabulary
            # GEMMs (unaligned 50257-element rows) through rocBLAS
            sp = self.DW_SPLITS.get(tag, 1)
            if sp > 1 and ct == F32 and Kd % sp == 0:
                calls.append(_Call(lib.mk_gemm_splitk, [st, _I(ab), _I64(M), _I64(N), _I64(Kd), a, _I64(a_ms),
                                                        _I64(a_ks), b, _I64(b_ks), _I64(b_ns), cptr, _I64(c_ms),
                                                        _I64(sp), ws], "mk_gemm_splitk " + tag))
                return
            if tag in self.BLAS_GEMMS:
                calls.append(_Call(lib.mk_gemm_blas, [st, _I(ab), _I(ct), _I64(1), _I64(M), _I64(N), _I64(Kd),
                                                      a, _I64(0), _I64(a_ms), _I64(a_ks), b, _I64(0), _I64(b_ks),
                                                      _I64(b_ns), cptr, _I64(0), _I64(c_ms), _F(1.0), _F(0.0)],
                                   "mk_gemm_blas " + tag))
                return
            if tag == "dhf":
                calls.append(_Call(lib.mk_gemm_splitk_typed, [st, _I(ab), _I(ct), _I64(M), _I64(N), _I64(Kd), a,
                                                              _I64(a_ms), _I64(a_ks), b, _I64(b_ks), _I64(b_ns), cptr,
                                                              _I64(c_ms), _I64(self.DHF_SPLITS), ws, _P(0), _I(0)],
                                   "mk_gemm_splitk_typed " + tag))
                return
            calls.append(_Call(lib.mk_gemm, [st, _I(ab), _I(ct), _I64(1), _I64(M), _I64(N), _I64(Kd),
                                             a, _I64(0), _I64(a_ms), _I64(a_ks), b, _I64(0), _I64(b_ks),
                                             _I64(b_ns), cptr, _I64(0), _I64(c_ms), bias or _P(0),
                                             _I(0 if bias is None else 1)], "mk_gemm " + tag))

        def add_rows(out, rows, cols, a, b=None, bias=None, tag="add"):
            """out = a (+ b) (+ bias broadcast over rows), one mk_add_rows pass"""
            calls.append(_Call(lib.mk_add_rows, [st, _I(BF16), _I64(rows), _I64(cols), a, b or _P(0),
                                                 bias or _P(0), out], "mk_add_rows " + tag))

        def layernorm(x, gname, bname, y):
            calls.append(_Call(lib.mk_layernorm, [st, _I(BF16), _I64(T), _I64(d), x, W(gname), W(bname),
                                                  _F(c.ln_eps), y], "mk_layernorm"))

        def add_layernorm(a, b, bias, ln, sum_out, y):
            """sum_out = a + b + bias, y = LayerNorm(sum_out) with ln's parameters"""
            calls.append(_Call(lib.mk_add_layernorm, [st, _I64(T), _I64(d), a, b, bias, W(ln + "_g"), W(ln + "_b"),
                                                      _F(c.ln_eps), sum_out, y], "mk_add_layernorm"))

        def colsum(x, rows, cols, out):
            calls.append(_Call(lib.mk_col_sum, [st, _I(BF16), _I64(rows), _I64(cols), x, out, ws], "mk_col_sum"))

        def ln_bwd(x, gname, dy, dres, dx, prefix, colsum_out):
            """dx = dres + LN'(dy), its LN parameter gradients and (when
            colsum_out is given) the column sums of dx in one pass"""
            calls.append(_Call(lib.mk_layernorm_bwd, [st, _I(BF16), _I64(T), _I64(d), x, W(gname), dy,
                                                      dres or _P(0), _F(c.ln_eps), dx, G(prefix + "_g"),
                                                      G(prefix + "_b"), colsum_out or _P(0), ws],
                               "mk_layernorm_bwd"))

        scale = 1.0 / math.sqrt(hd)
        # the MLP's products can take the GELU in their epilogues where the
        # tiled kernel takes the shapes (16-byte aligned rows, M, N >= 128, K >= 64)
        tiled_mlp = T >= 128 and F >= 128 and d >= 64 and F % 8 == 0 and d % 8 == 0
        # ---- forward
        calls.append(_Call(lib.mk_gather_rows, [st, _I64(V), _I64(d * 2), W("wte"), _I(S32), _I64(T),
                                                P(self.ids), P(self.x[0])], "mk_gather_rows"))
        # x0 += wpe broadcast over the batch: [B, S*d] + [S*d]
        add_rows(P(self.x[0]), B, S * d, P(self.x[0]), bias=W("wpe"), tag="pos")
        # LN1 of layer 0 stands alone; every later LayerNorm (LN1 of the next
        # layer, LN2, the final LN) is fused with the residual add before it
        layernorm(P(self.x[0]), "h0.ln1_g", "h0.ln1_b", P(self.h1[0]))
        for l in range(L):
            p = f"h{l}."
            gemm(BF16, BF16, T, 3 * d, d, P(self.h1[l]), d, 1, W(p + "w_qkv"), 3 * d, 1, P(self.qkv[l]), 3 * d,
                 tag="qkv", bias=W(p + "b_qkv"))
            q, k, v = (P(self.qkv[l], i * d) for i in range(3))
            strides_qkv = [_I64(S * 3 * d), _I64(hd), _I64(3 * d)]
            calls.append(_Call(lib.mk_sdpa_fwd, [st, _I64(B), _I64(H), _I64(S), _I64(S), _I64(hd),
                                                 q, *strides_qkv, k, *strides_qkv, v, *strides_qkv,
                                                 P(self.att[l]), _I64(S * d), _I64(hd), _I64(d),
                                                 _F(scale), _I(1), P(self.lse[l])], "mk_sdpa_fwd"))
            gemm(BF16, BF16, T, d, d, P(self.att[l]), d, 1, W(p + "w_o"), d, 1, P(self.tmp), d, tag="o")
            add_layernorm(P(self.x[l]), P(self.tmp), W(p + "b_o"), p + "ln2", P(self.xm[l]), P(self.h2[l]))
            if tiled_mlp and self.FUSE_GELU_FWD:
                # the up-projection, its bias and the GELU in one launch (the tiled
                # kernel's shapes): f = h2 w_fc + b_fc, kept for the backward, and
                # g = gelu_tanh(f) from the epilogue
                calls.append(_Call(lib.mk_gemm_bias_gelu, [st, _I(BF16), _I(BF16), _I64(T), _I64(F), _I64(d),
                                                           P(self.h2[l]), _I64(d), _I64(1), W(p + "w_fc"), _I64(F),
                                                           _I64(1), P(self.f[l]), _I64(F), W(p + "b_fc"), _I(1),
                                                           P(self.g[l]), _I64(F)], "mk_gemm_bias_gelu fc"))
            else:
                gemm(BF16, BF16, T, F, d, P(self.h2[l]), d, 1, W(p + "w_fc"), F, 1, P(self.f[l]), F, tag="fc")
                calls.append(_Call(lib.mk_bias_gelu, [st, _I64(T), _I64(F), P(self.f[l]), W(p + "b_fc"),
                                                      P(self.f[l]), P(self.g[l])], "mk_bias_gelu"))
            gemm(BF16, BF16, T, d, F, P(self.g[l]), F, 1, W(p + "w_pr"), d, 1, P(self.tmp), d, tag="proj")
            nxt, y = (f"h{l + 1}.ln1", P(self.h1[l + 1])) if l + 1 < L else ("lnf", P(self.hf))
            add_layernorm(P(self.xm[l]), P(self.tmp), W(p + "b_pr"), nxt, P(self.x[l + 1]), y)
        # logits = hf @ wteᵀ, then loss rows and dlogits (over the logits)
        Vp = self.vocab_pitch
        gemm(BF16, BF16, T, V, d, P(self.hf), d, 1, W("wte"), 1, d, P(self.logits), Vp, tag="logits")
        calls.append(_Call(lib.mk_softmax_xent_strided, [st, _I(BF16), _I(BF16), _I64(T), _I64(V), P(self.logits),
                                                         _I64(Vp), _I(S32), P(self.labels), _F(1.0 / T),
                                                         P(self.loss_rows), P(self.logits), _I64(Vp)],
                           "mk_softmax_xent_strided"))
        calls.append(_Call(lib.mk_row_reduce, [st, _I(F32), _I(F32), _I(0), _I64(1), _I64(T), P(self.loss_rows),
                                               _F(0.0), P(self.loss_sum)], "mk_row_reduce"))
        # ---- backward
        dlog = P(self.logits)
        gemm(BF16, BF16, T, d, V, dlog, Vp, 1, W("wte"), d, 1, P(self.dh), d, tag="dhf")
        gemm(BF16, F32, V, d, T, dlog, 1, Vp, P(self.hf), d, 1, G("wte"), d, tag="dwte")
        # the bias gradient of each residual projection is the column sum of
        # the residual-stream gradient, produced by the LayerNorm backward
        # that writes it
        ln_bwd(P(self.x[L]), "lnf_g", P(self.dh), None, P(self.dx), "lnf", G(f"h{L - 1}.b_pr"))
        for l in reversed(range(L)):
            p = f"h{l}."
            # MLP branch of x[l+1] = xm + proj(gelu(fc(ln2(xm))))
            gemm(BF16, F32, F, d, T, P(self.g[l]), 1, F, P(self.dx), d, 1, G(p + "w_pr"), d, tag="dw_pr")
            if tiled_mlp and self.FUSE_GELU_BWD:
                # dff = gelu'(f) * (dx w_prᵀ) and the fc bias gradient, the GELU
                # backward in the product's epilogue
                calls.append(_Call(lib.mk_gemm_gelu_bwd, [st, _I(BF16), _I64(T), _I64(F), _I64(d), P(self.dx), _I64(d),
                                                          _I64(1), W(p + "w_pr"), _I64(1), _I64(d), P(self.dff),
                                                          _I64(F), P(self.f[l]), _I64(F), G(p + "b_fc"), ws],
                                   "mk_gemm_gelu_bwd dg"))
            else:
                gemm(BF16, BF16, T, F, d, P(self.dx), d, 1, W(p + "w_pr"), 1, d, P(self.dff), F, tag="dg")
                calls.append(_Call(lib.mk_gelu_tanh_bwd_colsum, [st, _I(BF16), _I64(T), _I64(F), P(self.f[l]),
                                                                 P(self.dff), P(self.dff), G(p + "b_fc"), ws],
                                   "mk_gelu_tanh_bwd_colsum"))
            gemm(BF16, F32, d, F, T, P(self.h2[l]), 1, d, P(self.dff), F, 1, G(p + "w_fc"), F, tag="dw_fc")
            gemm(BF16, BF16, T, d, F, P(self.dff), F, 1, W(p + "w_fc"), 1, F, P(self.dh), d, tag="dh2")
            ln_bwd(P(self.xm[l]), p + "ln2_g", P(self.dh), P(self.dx), P(self.dx), p + "ln2", G(p + "b_o"))
            # attention branch of xm = x[l] + o(attn(ln1(x[l])))
            gemm(BF16, F32, d, d, T, P(self.att[l]), 1, d, P(self.dx), d, 1, G(p + "w_o"), d, tag="dw_o")
            gemm(BF16, BF16, T, d, d, P(self.dx), d, 1, W(p + "w_o"), 1, d, P(self.dh), d, tag="datt")
            q, k, v = (P(self.qkv[l], i * d) for i in range(3))
            dq, dk, dv = (P(self.dqkv, i * d) for i in range(3))
            sq = [_I64(S * 3 * d), _I64(hd), _I64(3 * d)]
            sd = [_I64(S * d), _I64(hd), _I64(d)]
            calls.append(_Call(lib.mk_sdpa_bwd, [st, _I64(B), _I64(H), _I64(S), _I64(S), _I64(hd),
                                                 q, *sq, k, *sq, v, *sq, P(self.att[l]), *sd, P(self.dh), *sd,
                                                 P(self.lse[l]), dq, *sq, dk, *sq, dv, *sq,
                                                 _F(scale), _I(1), ws], "mk_sdpa_bwd"))
            gemm(BF16, F32, d, 3 * d, T, P(self.h1[l]), 1, d, P(self.dqkv), 3 * d, 1, G(p + "w_qkv"), 3 * d,
                 tag="dw_qkv")
            colsum(P(self.dqkv), T, 3 * d, G(p + "b_qkv"))
            gemm(BF16, BF16, T, d, 3 * d, P(self.dqkv), 3 * d, 1, W(p + "w_qkv"), 1, 3 * d, P(self.dh), d,
                 tag="dh1")
            ln_bwd(P(self.x[l]), p + "ln1_g", P(self.dh), P(self.dx), P(self.dx), p + "ln1",
                   G(f"h{l - 1}.b_pr") if l > 0 else None)
        # embeddings: position gradient = sum over the batch; token gradient
        # scattered (in token order) into the head's embedding gradient
        colsum(P(self.dx), B, S * d, G("wpe"))
        calls.append(_Call(lib.mk_convert, [st, _I(BF16), _I(F32), _I64(T * d), P(self.dx), P(self.dx32)],
                           "mk_convert"))
        calls.append(_Call(lib.mk_scatter_add_rows, [st, _I(F32), _I64(V), _I64(d), G("wte"), _I(S32), _I64(T),
                                                     P(self.ids), P(self.dx32), G("wte"), ws],
                           "mk_scatter_add_rows"))
        self.n_fwd_bwd = len(calls)
        return calls

    # ------------------------------------------------------------------ running
    def set_batch(self, ids, labels):
        self.ids.copy_(torch.as_tensor(ids, dtype=torch.int32).reshape(-1))
        self.labels.copy_(torch.as_tensor(labels, dtype=torch.int32).reshape(-1))

    def forward_backward(self):
        """Loss (device tensor, mean over tokens) and all gradients in self.grad."""
        for call in self.calls:
            call()
        return self.loss_sum

    def set_step_scalars(self, t=None):
        """Advance the step count and write the step's scalar inputs (lr and
        the bias corrections bc1 = 1-b1^t, bc2 = 1-b2^t, host-computed in
        double and rounded to fp32: temp/dp_train.py:91-95) to the device."""
        self.t = self.t + 1 if t is None else t
        bc1, bc2 = 1 - self.b1 ** self.t, 1 - self.b2 ** self.t
        k = self.t % len(self._hyper_host)
        if self._hyper_done[k] is not None:
            self._hyper_done[k].synchronize()
        host = self._hyper_host[k]
        host[0], host[1], host[2] = self.lr, bc1, bc2
        with torch.cuda.stream(self.stream):
            self.hyper.copy_(host, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.stream)
        self._hyper_done[k] = ev

    def _adam_launch(self):
        rc = self.lib.mk_adam_update_dev(_P(self.stream.cuda_stream), self.n_flat, BF16, _P(self.param.data_ptr()),
                                         _P(self.master.data_ptr()), F32, _P(self.grad.data_ptr()),
                                         _P(self.m.data_ptr()), _P(self.v.data_ptr()), _P(self.hyper.data_ptr()),
                                         self.b1, self.b2, self.adam_eps)
        K._check(rc, "mk_adam_update_dev")

    def adam(self, t=None):
        """One Adam update of every parameter (temp/dp_train.py:71-75)."""
        self.set_step_scalars(t)
        self._adam_launch()

    def step(self):
        """forward + backward + Adam; returns the (pre-update) mean loss as a
        device tensor of one element (sum of loss rows / tokens)."""
        self.forward_backward()
        self.adam()
        return self.loss_sum

    def capture(self):
        """Record forward + backward + the Adam launch as one HIP graph on the
        step's stream (which must not be the default stream).  Run one eager
        step first: library handles are created on first use, outside any
        capture.  The graph reads the step scalars from device memory, so each
        replay() takes that step's lr and bias corrections."""
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(self.stream):
            with torch.cuda.graph(self.graph, stream=self.stream):
                for call in self.calls:
                    call()
                self._adam_launch()
        return self.graph

    def replay(self):
        """One training step by graph replay (after capture())."""
        self.set_step_scalars()
        with torch.cuda.stream(self.stream):
            self.graph.replay()
        return self.loss_sum

    def loss_value(self) -> float:
        return float(self.loss_sum.item()) / self.cfg.tokens
