"""C5 as one jitted module through the PJRT C API: the training step written
as StableHLO (mi355x_pjrt/train_hlo.py: loss, gradients by reverse mode, the
Adam update of temp/dp_train.py:67-76) compiled by jam and run with
PJRT_LoadedExecutable_Execute, against the float64 restatement
(oracle/gpt2_ref.py) on the reduced GPT-2 configuration of test_gpu_gpt2.py.

Tolerance: the module rounds the matrix-product operands to bf16 (fp32
accumulation, everything else fp32), so each gradient tensor is compared by
its relative L2 error against the float64 gradient of the same fp32
parameters (3e-2, as for the hand-scheduled step) and the loss to 2e-3
relative.  The Adam outputs are checked against float64 Adam applied to the
module's own gradients, to fp32 rounding."""

import numpy as np
import pytest

from mi355x_pjrt import gpt2, pjrt, train_hlo
from oracle import gpt2_ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def client():
    p = pjrt.Plugin()
    c = p.client()
    if c.device_kind(c.devices()[0]) != "MI355X":
        pytest.skip("no device")
    yield c
    c.close()


def _params(cfg, seed=0):
    p = gpt2.init_params(cfg, seed)
    rng = np.random.default_rng(seed + 1)
    for n in p:  # non-trivial LayerNorm parameters and biases, so every gradient path is exercised
        leaf = n.split(".")[-1]
        if leaf.endswith("_g"):
            p[n] = (1 + 0.1 * rng.standard_normal(p[n].shape)).astype(np.float32)
        elif leaf.startswith("b_") or leaf.endswith("_b"):
            p[n] = (0.02 * rng.standard_normal(p[n].shape)).astype(np.float32)
    return p


def _step(client, cfg, params, m, v, ids, labels, lr, t, b1=0.9, b2=0.999):
    text = train_hlo.gpt2_train_step(cfg, return_grads=True)
    e = client.compile(text)
    names = [n for n, _ in cfg.param_shapes()]
    host = ([params[n] for n in names] + [m[n] for n in names] + [v[n] for n in names] +
            [ids.astype(np.int32), labels.astype(np.int32),
             np.float32(lr), np.float32(1 / (1 - b1 ** t)), np.float32(1 / (1 - b2 ** t))])
    bufs = [client.put(np.asarray(a)) for a in host]
    outs = e.execute(bufs)
    res = [o.to_numpy() for o in outs]
    for b in bufs + outs:
        b.destroy()
    e.destroy()
    k = len(names)
    loss = float(res[0])
    split = lambda lo: {n: res[lo + i] for i, n in enumerate(names)}  # noqa: E731
    return loss, split(1), split(1 + k), split(1 + 2 * k), split(1 + 3 * k)


def test_gpt2_jitted_step_small_vs_float64(client):
    cfg = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    print("case: jitted gpt2 step L2 d128 H2 S128 B2 V257 through PJRT Execute", flush=True)
    params = _params(cfg)
    zeros = {n: np.zeros_like(a) for n, a in params.items()}
    rng = np.random.default_rng(5)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    labels = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    lr = 1e-3
    loss, new_p, new_m, new_v, grads = _step(client, cfg, params, zeros, zeros, ids, labels, lr, 1)
    ref_loss, ref_grads = gpt2_ref.loss_and_grads(params, ids, labels, cfg.n_layer, cfg.n_head)
    assert abs(loss - ref_loss) < 2e-3 * abs(ref_loss), (loss, ref_loss)
    worst = {n: float(np.linalg.norm(grads[n] - ref_grads[n]) / max(np.linalg.norm(ref_grads[n]), 1e-30))
             for n in grads}
    bad = {n: e for n, e in worst.items() if e > 3e-2}
    assert not bad, bad
    for n in params:
        want_p, want_m, want_v = gpt2_ref.adam(params[n].astype(np.float64), grads[n].astype(np.float64),
                                               0.0, 0.0, 1, lr)
        np.testing.assert_allclose(new_m[n], want_m, rtol=1e-6, atol=1e-12, err_msg=n)
        np.testing.assert_allclose(new_v[n], want_v, rtol=1e-5, atol=1e-18, err_msg=n)
        np.testing.assert_allclose(new_p[n], want_p, rtol=0, atol=2e-6 + lr * 1e-5, err_msg=n)


def test_gpt2_jitted_steps_descend(client):
    """Three steps of the jitted module with its own Adam state: the loss on
    a fixed batch goes down."""
    cfg = gpt2.GPT2Config(n_layer=2, d_model=128, n_head=2, seq=128, batch=2, vocab=257)
    params = _params(cfg, seed=3)
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    rng = np.random.default_rng(9)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    losses = []
    for t in (1, 2, 3):
        loss, params, m, v, _ = _step(client, cfg, params, m, v, ids, np.roll(ids, -1, axis=1), 3e-3, t)
        losses.append(loss)
    assert np.isfinite(losses).all() and losses[2] < losses[0], losses


def test_gpt2_jitted_step_c5_full_size(client):
    """The benchmark configuration (12 layers, d 768, B 8, S 1024, V 50257)
    as one jitted module through Execute, against the hand-scheduled step
    (GPT2TrainStep: the same kernels launched from Python) on the same fp32
    parameters and batch:
      - loss within 0.5 of ln V at random init, and within 2e-3 relative of
        the hand-scheduled step's;
      - every output finite;
      - each gradient within 3e-2 relative L2 of the hand-scheduled step's
        (both round the products' operands to bf16);
      - gradient signs agree on at least 99% of the elements whose |g| is
        above 5% of the tensor's rms (clear of bf16 rounding noise);
      - the updated parameters: at t = 1 Adam moves each by
        lr * g / (|g| + eps), so where both gradients have one sign and
        |g| > 1e-5 (1000 eps) the new parameters agree to 1e-3 lr plus fp32
        rounding."""
    import torch

    cfg = gpt2.GPT2Config()
    print("case: jitted gpt2 step C5 full size through PJRT Execute vs GPT2TrainStep", flush=True)
    params = gpt2.init_params(cfg, 0)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    labels = np.roll(ids, -1, axis=1)
    zeros = {n: np.zeros_like(a) for n, a in params.items()}
    lr = 3e-4
    loss, new_p, new_m, new_v, grads = _step(client, cfg, params, zeros, zeros, ids, labels, lr, 1)
    assert abs(loss - np.log(cfg.vocab)) < 0.5, loss
    for out in (new_p, new_m, new_v, grads):
        bad = [n for n, a in out.items() if not np.isfinite(a).all()]
        assert not bad, bad

    step = gpt2.GPT2TrainStep(cfg, params=params, lr=lr)
    step.set_batch(ids, labels)
    step.step()
    torch.cuda.synchronize()
    h_loss = step.loss_value()
    h_grad = step.params_numpy(step.grad)
    h_p = step.params_numpy(step.master)
    print(f"loss jitted {loss:.6f}  hand-scheduled {h_loss:.6f}", flush=True)
    assert abs(loss - h_loss) <= 2e-3 * abs(h_loss)
    worst_g, worst_p, worst_agree = 0.0, 0.0, 1.0
    for n in params:
        g, hg = grads[n].astype(np.float64), h_grad[n].astype(np.float64)
        rel = float(np.linalg.norm(g - hg) / max(np.linalg.norm(hg), 1e-30))
        worst_g = max(worst_g, rel)
        assert rel < 3e-2, (n, rel)
        # signs are compared where |g| is well above both steps' rounding
        # noise (bf16 operands: about 1% of the tensor's rms)
        big = np.abs(hg) > 0.05 * np.sqrt(np.mean(hg ** 2))
        same = np.sign(g) == np.sign(hg)
        agree = float(np.mean(same[big])) if big.any() else 1.0
        worst_agree = min(worst_agree, agree)
        assert agree >= 0.99, (n, agree)
        # where both |g| exceed 1e-5 = 1000 eps with one sign, each update is
        # sign(g) lr (1 - eps / |g|): the two agree to 1e-3 lr
        sel = (np.abs(g) > 1e-5) & (np.abs(hg) > 1e-5) & same
        d = np.abs(new_p[n].astype(np.float64) - h_p[n].astype(np.float64))[sel]
        tol = 1e-3 * lr + 2.0 ** -22 * np.abs(params[n].astype(np.float64))[sel]
        if d.size:
            worst_p = max(worst_p, float((d / tol).max()))
        if not np.all(d <= tol):
            k = np.flatnonzero(sel)[np.argmax(d - tol)]
            print(f"{n}: {int((d > tol).sum())} of {d.size} elements out of bound; worst at {k}: g {g.flat[k]:.6e} "
                  f"hand g {hg.flat[k]:.6e} p0 {params[n].flat[k]:.8e} jitted p {new_p[n].flat[k]:.8e} "
                  f"hand p {h_p[n].flat[k]:.8e}", flush=True)
        assert np.all(d <= tol), (n, float(d.max()))
    print(f"worst gradient rel L2 {worst_g:.3e}, worst sign agreement {worst_agree:.5f}, "
          f"worst parameter diff / bound {worst_p:.3f}", flush=True)
