"""float64 restatement of the C5 training step (oracle; test infrastructure only).

The computation the reference's loop jits per rank (temp/dp_train.py:67-76:
jax.value_and_grad of the mean loss, then the Adam update of lines 71-75) for
a pre-LayerNorm GPT-2 decoder with tied embeddings, GELU(tanh) MLP and causal
attention, in float64 on the CPU with torch autograd as the differentiator
(an implementation independent of the kernels under test).  Parameters are
taken at the values the GPU step uses (its bf16 working copy), so the
comparison isolates the rounding of the bf16 activations.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def forward_loss(params: dict, ids: np.ndarray, labels: np.ndarray, n_layer: int, n_head: int,
                 ln_eps: float = 1e-5):
    """Mean softmax cross-entropy over all tokens; params are float64 torch
    tensors (requires_grad as the caller wants)."""
    B, S = ids.shape
    wte, wpe = params["wte"], params["wpe"]
    d = wte.shape[1]
    hd = d // n_head
    ids_t = torch.as_tensor(ids, dtype=torch.long)
    x = wte[ids_t] + wpe[:S][None]
    causal = torch.ones(S, S, dtype=torch.bool).tril()

    def ln(t, g, b):
        return torch.nn.functional.layer_norm(t, (d,), g, b, ln_eps)

    for l in range(n_layer):
        p = lambda n: params[f"h{l}.{n}"]  # noqa: E731
        h = ln(x, p("ln1_g"), p("ln1_b"))
        qkv = h @ p("w_qkv") + p("b_qkv")
        q, k, v = (qkv[..., i * d:(i + 1) * d].reshape(B, S, n_head, hd).transpose(1, 2) for i in range(3))
        s = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
        s = s.masked_fill(~causal, float("-inf"))
        a = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B, S, d)
        x = x + a @ p("w_o") + p("b_o")
        h2 = ln(x, p("ln2_g"), p("ln2_b"))
        f = torch.nn.functional.gelu(h2 @ p("w_fc") + p("b_fc"), approximate="tanh")
        x = x + f @ p("w_pr") + p("b_pr")
    hf = ln(x, params["lnf_g"], params["lnf_b"])
    logits = hf @ wte.T
    return torch.nn.functional.cross_entropy(logits.reshape(B * S, -1), torch.as_tensor(labels, dtype=torch.long)
                                             .reshape(-1))


def loss_and_grads(params_np: dict, ids, labels, n_layer, n_head, ln_eps=1e-5):
    """(loss, {name: grad}) in float64."""
    params = {n: torch.tensor(np.asarray(a, dtype=np.float64), requires_grad=True) for n, a in params_np.items()}
    loss = forward_loss(params, ids, labels, n_layer, n_head, ln_eps)
    loss.backward()
    return float(loss.detach()), {n: t.grad.numpy() for n, t in params.items()}


def adam(p, g, m, v, t, lr, b1=0.9, b2=0.999, eps=1e-8):
    """temp/dp_train.py:71-75 in float64 (bias corrections from the step t)."""
    bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    return p - lr * (m / bc1) / (np.sqrt(v / bc2) + eps), m, v
