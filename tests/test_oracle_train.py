"""Pins the oracle's training path (Backward, HeadBackward, layerNormBwd,
geluGrad, the RoPE inverse, attnBwd and AdamW) before it is trusted as the
checker of the device backward: against the reference's own PyTorch fixture
(gradients g.* of tiny_ref.safetensors), against central finite differences of
the oracle's own forward, and against AdamW's closed form at step 1."""
import math

import numpy as np
import pytest

import oracle
from conftest import rel_err, tiny_config, tiny_weights


def _tiny(tiny_ref):
    from decide_amd.nn import build_sequence, tensor_shapes

    tensors, meta = tiny_ref
    cfg = tiny_config(meta)
    weights = tiny_weights(tensors, cfg)
    model = oracle.OracleModel(cfg, weights)
    batch = [build_sequence(s["ids"], meta["mask_id"], s["independent"]) for s in meta["seqs"]]
    targets = [s["target"] for s in meta["seqs"]]
    return tensors, cfg, weights, model, batch, targets, tensor_shapes(cfg)


@pytest.mark.parametrize("train_from", [0, 2])
def test_backward_matches_pytorch_fixture(tiny_ref, train_from):
    """TestForwardBackwardMatchesPyTorch (internal/nn/nn_test.go:105-160):
    logits rel <= 1e-4, loss within 1e-4, every trainable gradient rel <= 2e-3
    against the fixture; frozen tensors (layers below trainFrom, and the
    embeddings when trainFrom > 0) receive exactly zero."""
    tensors, cfg, _, model, batch, targets, shapes = _tiny(tiny_ref)
    oracle.set_workers(4)
    logits = model.forward_train(batch, train_from)
    assert rel_err(logits, tensors["logits"]) <= 1e-4
    loss, dl = oracle.loss_and_grad(logits, batch, targets)
    assert abs(loss - float(tensors["loss"][0])) <= 1e-4
    g = model.zeros_like()
    model.backward(dl, g, train_emb=True)
    for name, shape in shapes.items():
        got = g.get(name, int(np.prod(shape)))
        frozen = any(name.startswith(f"model.layers.{l}.") for l in range(train_from))
        if train_from > 0 and (frozen or name.startswith("model.embeddings.")):
            assert np.all(got == 0), name
            continue
        assert rel_err(got, tensors["g." + name].reshape(-1)) <= 2e-3, name


def test_backward_matches_finite_differences():
    """d(sum_r c_r logit_r)/dw by central differences of the oracle's forward,
    for sampled entries of every tensor kind, on a random 3-layer model with a
    global and two local layers (window 4), an independent-options sequence
    and a plain one. Tolerance 3e-2 relative (fp32 forward, step 3e-3)."""
    from decide_amd.nn import Config, build_sequence, tensor_shapes

    cfg = Config(hidden=32, intermediate=48, heads=4, layers=3, vocab=40, eps=1e-5, half_window=4,
                 global_theta=160000.0, local_theta=10000.0,
                 layer_types=["full_attention", "sliding_attention", "sliding_attention"])
    rng = np.random.default_rng(11)
    shapes = tensor_shapes(cfg)
    w = {}
    for name, shape in shapes.items():
        if len(shape) == 2 or name.endswith("bias"):
            w[name] = (rng.standard_normal(shape) * 0.2).astype(np.float32)
        else:
            w[name] = (1 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
    mask = 39
    s0 = [1] + list(rng.integers(3, 38, 9)) + [2, mask] + list(rng.integers(3, 38, 4)) + [mask] + \
        list(rng.integers(3, 38, 5)) + [mask, 7, 8, 2]
    s1 = [1] + list(rng.integers(3, 38, 12)) + [mask, 5, 6, mask, 9, 2]
    batch = [build_sequence(s0, mask, True), build_sequence(s1, mask, False)]
    R = sum(len(s.mask_pos) for s in batch)
    coef = rng.standard_normal(R).astype(np.float32)

    def objective(ws):
        m = oracle.OracleModel(cfg, ws)
        return float(np.dot(m.forward(batch).astype(np.float64), coef.astype(np.float64)))

    model = oracle.OracleModel(cfg, w)
    model.forward_train(batch, 0)
    g = model.zeros_like()
    model.backward(coef, g, train_emb=True)
    h = 3e-3
    checked, want_checked = 0, 0
    for name, shape in shapes.items():
        n = int(np.prod(shape))
        grad = g.get(name, n)
        flat = w[name].reshape(-1)
        if name == "model.embeddings.tok_embeddings.weight":
            used = sorted(set(s0) | set(s1))
            picks = [used[0] * cfg.hidden + 3, used[-1] * cfg.hidden + 17]
            assert np.all(grad.reshape(cfg.vocab, cfg.hidden)[[i for i in range(cfg.vocab) if i not in used]] == 0)
        else:
            picks = [int(i) for i in np.argsort(-np.abs(grad))[:2]]
        want_checked += len(picks)
        for i in picks:
            wp = dict(w)
            wm = dict(w)
            fp, fm = flat.copy(), flat.copy()
            fp[i] += h
            fm[i] -= h
            wp[name] = fp.reshape(shape)
            wm[name] = fm.reshape(shape)
            fd = (objective(wp) - objective(wm)) / (2 * h)
            assert abs(fd - grad[i]) <= 3e-2 * max(abs(fd), 1e-2), (name, i, fd, grad[i])
            checked += 1
    assert checked == want_checked >= 2 * len(shapes) - 1


def test_gelu_grad_and_rope_inverse_closed_forms():
    """geluGrad(0) = 1/2, -> 1 for large x, -> 0 for very negative x; the
    inverse rotation undoes the forward one (up to rounding)."""
    _ = oracle.lib()
    cs, sn = oracle.rope_tables(np.array([0, 3, 41, 500], np.int32), 64, 10000.0)
    T, H, heads, D = 4, 128, 2, 64
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal(T * 3 * H).astype(np.float32)
    x = qkv.copy()
    oracle.apply_rope(x, T, H, heads, D, cs, sn)
    oracle.lib().orc_apply_rope_inverse(x, T, H, heads, D, cs, sn)
    assert np.allclose(x, qkv, atol=1e-5)
    assert oracle.lib().orc_gelu_grad(0.0) == 0.5
    assert oracle.lib().orc_gelu_grad(12.0) == 1.0
    assert abs(oracle.lib().orc_gelu_grad(-12.0)) < 1e-20
    # derivative of x*Phi(x): Phi(1) + phi(1)
    assert abs(oracle.lib().orc_gelu_grad(1.0) - (0.8413447460685429 + 0.24197072451914337)) < 1e-6


def test_adamw_step_one_closed_form(tiny_ref):
    """Update (internal/train/optim.go:94-145) at step 1 from zero moments:
    m = (1-b1) g', v = (1-b2) g'^2 with g' = g * scale, and
    p -= lr * g'/(|g'| + eps) + wd*lr*p (decay for 2-D tensors except the
    token embeddings; the scorer uses headLR). Frozen tensors are untouched.
    GradNorm = sqrt(sum g^2) over trainable tensors."""
    tensors, cfg, weights, model, batch, targets, shapes = _tiny(tiny_ref)
    logits = model.forward_train(batch, 1)
    _, dl = oracle.loss_and_grad(logits, batch, targets)
    g = model.zeros_like()
    model.backward(dl, g, train_emb=False)
    opt = oracle.OracleAdamW(model, g, weight_decay=0.01, train_from=1, train_emb=False)
    grads = {n: g.get(n, int(np.prod(s))) for n, s in shapes.items()}
    trainable = {n for n in shapes if not n.startswith("model.embeddings.") and not n.startswith("model.layers.0.")}
    gn = math.sqrt(sum(float((grads[n].astype(np.float64) ** 2).sum()) for n in trainable))
    assert abs(opt.grad_norm() - gn) <= 1e-12 * max(gn, 1)
    lr, head_lr, scale = 1e-3, 3e-3, 0.5
    opt.update(lr, head_lr, scale)
    for name, shape in shapes.items():
        n = int(np.prod(shape))
        p0 = weights[name].reshape(-1).astype(np.float64)
        p1 = model.get(name, n).astype(np.float64)
        if name not in trainable:
            assert np.array_equal(p1, p0), name
            continue
        rate = head_lr if name.startswith("scorer.") else lr
        wd = 0.01 * rate if (len(shape) == 2 and name != "model.embeddings.tok_embeddings.weight") else 0.0
        gs = grads[name].astype(np.float64) * scale
        want = p0 - (rate * gs / (np.abs(gs) + 1e-8) + wd * p0)
        assert np.allclose(p1, want, rtol=0, atol=2e-6 * max(1.0, float(np.abs(p0).max()))), name
        m = opt.moment(name, 0, n).astype(np.float64)
        assert np.allclose(m, 0.1 * gs, rtol=1e-5, atol=1e-12), name
