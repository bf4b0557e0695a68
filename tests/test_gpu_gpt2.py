"""C5 end to end: the GPT-2 training step on the mk_* kernels against the
float64 restatement (oracle/gpt2_ref.py) on a reduced configuration, and the
full-size step for finiteness / loss descent.

Tolerance: the GPU step keeps activations in bf16 (8 significant bits), so
each gradient tensor is compared by its relative L2 error against the
float64 gradient of the same bf16-valued parameters; the loss to 2e-3
relative.  The Adam update is checked against float64 Adam applied to the
GPU's own gradients (so it isolates the optimizer), to fp32 rounding."""

import numpy as np
import pytest
import torch

from oracle import gpt2_ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def G(cuda):
    from mi355x_pjrt import gpt2

    return gpt2


def _small(G):
    return G.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)


def _params(G, cfg, seed=0):
    p = G.init_params(cfg, seed)
    rng = np.random.default_rng(seed + 1)
    for n in p:  # non-trivial LayerNorm parameters and biases, so every gradient path is exercised
        leaf = n.split(".")[-1]
        if leaf.endswith("_g"):
            p[n] = (1 + 0.1 * rng.standard_normal(p[n].shape)).astype(np.float32)
        elif leaf.startswith("b_") or leaf.endswith("_b"):
            p[n] = (0.02 * rng.standard_normal(p[n].shape)).astype(np.float32)
    return p


def test_gpt2_step_small_vs_float64(G):
    cfg = _small(G)
    print("case: gpt2 small L2 d128 H2 S128 B2 V257", flush=True)
    step = G.GPT2TrainStep(cfg, params=_params(G, cfg), lr=1e-3)
    rng = np.random.default_rng(5)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    labels = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    step.set_batch(ids, labels)
    step.forward_backward()
    torch.cuda.synchronize()
    loss = step.loss_value()
    bf_params = step.params_numpy(step.param)  # the bf16 values the step used
    ref_loss, ref_grads = gpt2_ref.loss_and_grads(bf_params, ids, labels, cfg.n_layer, cfg.n_head)
    assert abs(loss - ref_loss) < 2e-3 * abs(ref_loss), (loss, ref_loss)
    grads = step.params_numpy(step.grad)
    worst = {}
    for n, g in grads.items():
        r = ref_grads[n]
        worst[n] = float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))
    bad = {n: e for n, e in worst.items() if e > 3e-2}
    assert not bad, bad
    # Adam on the GPU's own gradients, against float64 Adam
    master0 = step.params_numpy(step.master)
    step.adam()
    torch.cuda.synchronize()
    master1 = step.params_numpy(step.master)
    for n in master0:
        want, _, _ = gpt2_ref.adam(master0[n].astype(np.float64), grads[n].astype(np.float64), 0.0, 0.0, 1, 1e-3)
        np.testing.assert_allclose(master1[n], want, rtol=0, atol=2e-6 + 1e-3 * 1e-5)
    assert torch.equal(step.param, step.master.bfloat16())


def test_gpt2_small_training_descends(G):
    cfg = _small(G)
    step = G.GPT2TrainStep(cfg, params=_params(G, cfg, seed=3), lr=3e-3)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    step.set_batch(ids, np.roll(ids, -1, axis=1))
    losses = []
    for _ in range(12):
        step.step()
        losses.append(step.loss_value())
    assert all(np.isfinite(losses))
    assert losses[-1] < losses[0] - 0.5, losses


def test_gpt2_c5_full_step_finite(G):
    """The benchmark configuration: one step runs, the loss starts at
    about ln(vocab) for random init and every gradient is finite."""
    cfg = G.GPT2Config()
    print("case: gpt2 C5 full size one step", flush=True)
    step = G.GPT2TrainStep(cfg, seed=0)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    step.set_batch(ids, np.roll(ids, -1, axis=1))
    step.step()
    torch.cuda.synchronize()
    loss = step.loss_value()
    assert abs(loss - np.log(cfg.vocab)) < 0.5, loss
    assert bool(torch.isfinite(step.grad).all())
    assert bool(torch.isfinite(step.master).all())


def test_gpt2_graph_replay_matches_eager(G):
    """The step captured as a HIP graph and replayed (with eager work and
    host synchronisation between replays) reproduces eager steps: same
    losses, same parameters; lr and the bias corrections of every step come
    from the device buffer the replay reads."""
    cfg = _small(G)
    rng = np.random.default_rng(21)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    labels = np.roll(ids, -1, axis=1)
    params = _params(G, cfg, seed=4)
    eager = G.GPT2TrainStep(cfg, params=params, lr=2e-3, stream=torch.cuda.Stream())
    graphed = G.GPT2TrainStep(cfg, params=params, lr=2e-3, stream=torch.cuda.Stream())
    for st in (eager, graphed):
        st.set_batch(ids, labels)
    eager.step()
    graphed.step()  # eager warm-up step (library handles), also step 1
    graphed.capture()
    for i in range(3):
        eager.step()
        graphed.replay()
        torch.cuda.synchronize()
        junk = torch.randn(1000, device="cuda").sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        assert float(junk) == float(junk)
        le, lg = eager.loss_value(), graphed.loss_value()
        assert abs(le - lg) <= 1e-6 * abs(le), (i, le, lg)
        np.testing.assert_allclose(graphed.master.cpu().numpy(), eager.master.cpu().numpy(), rtol=0, atol=1e-6)
    assert graphed.t == eager.t == 4
