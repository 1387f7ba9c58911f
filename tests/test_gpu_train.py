"""Training parity on the GPU: dn_forward_train / dn_backward / dn_adamw_step
through the C ABI against the CPU oracle's restatement of nn.Forward,
nn.Backward and AdamW (itself pinned to the reference's PyTorch gradients in
test_oracle_train.py).

Bars: logits as the forward tests (fp32 |dlogit| <= 1e-4 (1 + |logit|));
every gradient tensor within relErr (nn_test.go:95-103) <= 5e-4 in the fp32
validation mode and <= 1e-1 in bf16 (bf16 operands, fp32 accumulation), the
median over tensors <= 1e-4 / 5e-2, and its norm within 1e-5 / 1.5e-2 and
direction within 1 - cos <= 1e-8 / 5e-3 of the oracle's; the
same dlogits drive both sides so the backward is compared alone. AdamW is
checked against its closed form and against the oracle's AdamW fed the
device's gradients (fp32 arithmetic on both sides, same order)."""
import os

import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

WORKERS = max(1, min(16, os.cpu_count() or 1))
# fp32: rounding level (the scorer norm-bias gradient is a sum over rows of
# terms that cancel, since softmax cross-entropy gradients sum to zero per
# sequence; relErr's 1e-4 floor then measures absolute noise of ~1e-8).
# bf16: bf16 activations and GEMM / attention operands (the oracle gets the
# same bf16-rounded projection weights). Measured on ModernBERT-base: the
# MLP-output weight gradients 5-6.5%, QKV 1.4-1.8%, median 3.3%, the same at
# layer 21 as at layer 0 (no compounding through depth); an indexing or sign
# error gives O(1).
GRAD_TOL = {"fp32": 5e-4, "bf16": 1e-1}
GRAD_MEDIAN_TOL = {"fp32": 1e-4, "bf16": 5e-2}
# Per tensor, the gradient's norm and direction: bf16 rounding noise is
# unbiased elementwise and largely averages out of both, so these bars are
# far tighter than the elementwise relErr and catch a scale or sign error
# confined to one tensor (a 2% mis-scaling passes relErr <= 0.1). Measured
# over the small, medium and ModernBERT-base tests: |norm ratio - 1| <= 2.8e-6
# (fp32) / 8.8e-3 (bf16, the norm weights), 1 - cos <= 2.3e-10 / 1.9e-3 (bf16,
# Wi).
NORM_TOL = {"fp32": 1e-5, "bf16": 1.5e-2}
COS_TOL = {"fp32": 1e-8, "bf16": 5e-3}


def small_cfg(layers=3):
    from decide_amd.nn import Config

    types = ["full_attention", "sliding_attention", "sliding_attention"] * 3
    return Config(hidden=256, intermediate=384, heads=4, layers=layers, vocab=400, half_window=8,
                  layer_types=types[:layers])


def train_batch(vocab, mask_id, seed=0, specs=None):
    """Independent-option sequences and a plain one, lengths across the
    32/64/128-token tile edges; options of a few tokens each."""
    from decide_amd.nn import build_sequence

    rng = np.random.default_rng(seed)
    specs = specs or [(20, [5, 6, 7], True), (100, [10, 12], False), (150, [20, 20, 21], True), (9, [1, 3], True)]
    out = []
    for prem, opts, indep in specs:
        ids = [1] + list(rng.integers(3, mask_id, size=prem - 2)) + [2]
        for ln in opts:
            ids += [mask_id] + list(rng.integers(3, mask_id, size=ln - 1))
        ids.append(2)
        out.append(build_sequence(np.array(ids, np.int32), mask_id, independent=indep))
    return out


def weights_for(cfg, seed=3, std=0.05):
    from decide_amd.synth import random_weights

    w = random_weights(cfg, seed=seed, std=std)
    rng = np.random.default_rng(seed + 1)
    for name in w:  # norm weights and biases away from 1 / 0 so their gradients matter
        if name.endswith("norm.weight"):
            w[name] = (1 + 0.1 * rng.standard_normal(w[name].shape)).astype(np.float32)
        elif name.endswith(".bias"):
            w[name] = (0.05 * rng.standard_normal(w[name].shape)).astype(np.float32)
    return w


PROJ = ("attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight")


def bf16_round(a):
    """Round-to-nearest-even to bfloat16, widened back to float32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(np.shape(a))


def effective_weights(w, prec):
    """The weights the device computes with: in bf16 the four projection
    matrices are rounded to bfloat16 at upload."""
    if prec != "bf16":
        return w
    return {n: (bf16_round(a) if n.endswith(PROJ) else a) for n, a in w.items()}


def oracle_grads(cfg, w, batch, train_from=0, train_emb=True, seed=5):
    from decide_amd.nn import tensor_shapes

    oracle.set_workers(WORKERS)
    m = oracle.OracleModel(cfg, w)
    logits = m.forward_train(batch, train_from)
    rng = np.random.default_rng(seed)
    targets = [int(rng.integers(0, len(s.mask_pos))) for s in batch]
    _, dl = oracle.loss_and_grad(logits, batch, targets)
    g = m.zeros_like()
    m.backward(dl, g, train_emb=train_emb)
    grads = {n: g.get(n, int(np.prod(s))).reshape(s) for n, s in tensor_shapes(cfg).items()}
    return logits, dl, grads


def frozen(name, train_from, train_emb):
    if name == "model.embeddings.tok_embeddings.weight":
        return not train_emb or train_from > 0
    if name == "model.embeddings.norm.weight":
        return train_from > 0
    return any(name.startswith(f"model.layers.{l}.") for l in range(train_from))


def norm_and_direction(got, want):
    """|norm ratio - 1| and 1 - cosine of two gradient tensors (float64)."""
    g = np.asarray(got, np.float64).ravel()
    w = np.asarray(want, np.float64).ravel()
    ng, nw = np.linalg.norm(g), np.linalg.norm(w)
    if nw == 0.0:
        return (0.0 if ng == 0.0 else np.inf), 0.0
    return abs(ng / nw - 1.0), 1.0 - float(g @ w) / (ng * nw + 1e-300)


def check_grads(eng, want, prec, train_from=0, train_emb=True, label=""):
    worst, worst_name, errs = 0.0, "", []
    worst_norm, worst_cos = (0.0, ""), (0.0, "")
    for name, g_want in want.items():
        got = eng.download(name, "grad")
        if frozen(name, train_from, train_emb):
            assert np.all(got == 0), name
            continue
        if name == "model.embeddings.tok_embeddings.weight" and not train_emb:
            continue
        e = rel_err(got, g_want)
        errs.append(e)
        if e > worst:
            worst, worst_name = e, name
        assert np.all(np.isfinite(got)), name
        assert e <= GRAD_TOL[prec], (label, prec, name, e)
        dn, dc = norm_and_direction(got, g_want)
        if np.linalg.norm(g_want) > 1e-6:  # tensors whose gradient is rounding noise have no direction to check
            if dn > worst_norm[0]:
                worst_norm = (dn, name)
            if dc > worst_cos[0]:
                worst_cos = (dc, name)
            assert dn <= NORM_TOL[prec] and dc <= COS_TOL[prec], (label, prec, name, dn, dc)
    print(f"{label} {prec}: worst |norm ratio - 1| {worst_norm[0]:.3g} ({worst_norm[1]}), "
          f"worst 1 - cos {worst_cos[0]:.3g} ({worst_cos[1]})", flush=True)
    if os.environ.get("DN_GRAD_REPORT"):
        for name in want:
            if name.startswith("model.layers.") and name.endswith(("Wqkv.weight", "mlp.Wo.weight")):
                print(f"  {name}: {rel_err(eng.download(name, 'grad'), want[name]):.3g}", flush=True)
    med = float(np.median(errs))
    print(f"{label} {prec}: grad relErr worst {worst:.3g} ({worst_name}), median {med:.3g} over {len(errs)} "
          f"tensors", flush=True)
    assert med <= GRAD_MEDIAN_TOL[prec], (label, prec, med)
    return worst


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_backward_matches_oracle_small(prec):
    from decide_amd.train import TrainEngine

    cfg = small_cfg()
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1)
    print(f"case: small backward {prec}, T={sum(len(s.ids) for s in batch)}", flush=True)
    want_logits, dl, want = oracle_grads(cfg, effective_weights(w, prec), batch)
    with TrainEngine(cfg, w, precision=prec) as eng:
        logits = eng.forward(batch)
        if prec == "fp32":
            assert np.all(np.abs(logits.astype(np.float64) - want_logits) <= 1e-4 * (1 + np.abs(want_logits)))
        eng.backward(dl)
        check_grads(eng, want, prec, label="small")


def test_backward_duplicate_mask_positions_fp32():
    """Two [MASK] rows naming the same token (stage_batch accepts repeated
    mask positions): their scores and head gradients both count, and the
    reference copies the rows' gradients into dcur in row order, so the last
    such row's gradient is the one that flows into the encoder
    (backward.go:30-33). The target sits on the first duplicate, so the two
    rows' dlogits differ (p - 1 against p) and a wrong winner shows up in every
    encoder gradient."""
    from decide_amd.nn import Sequence
    from decide_amd.train import TrainEngine

    cfg = small_cfg(2)
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1, specs=[(20, [5, 6, 7], True), (30, [4, 4], False)])
    s0 = batch[0]
    mp = np.array([s0.mask_pos[0], s0.mask_pos[1], s0.mask_pos[2], s0.mask_pos[0]], np.int32)
    batch[0] = Sequence(ids=s0.ids, pos=s0.pos, opt=s0.opt, mask_pos=mp)
    print(f"case: duplicate mask positions fp32, T={sum(len(s.ids) for s in batch)}", flush=True)
    oracle.set_workers(WORKERS)
    m = oracle.OracleModel(cfg, w)
    want_logits = m.forward_train(batch, 0)
    _, dl = oracle.loss_and_grad(want_logits, batch, [0, 1])
    assert dl[0] != dl[3]
    g = m.zeros_like()
    m.backward(dl, g, train_emb=True)
    from decide_amd.nn import tensor_shapes

    want = {n: g.get(n, int(np.prod(sh))).reshape(sh) for n, sh in tensor_shapes(cfg).items()}
    with TrainEngine(cfg, w, precision="fp32") as eng:
        logits = eng.forward(batch)
        assert logits[0] == logits[3]
        assert np.all(np.abs(logits.astype(np.float64) - want_logits) <= 1e-4 * (1 + np.abs(want_logits)))
        eng.backward(dl)
        check_grads(eng, want, "fp32", label="duplicate mask positions")


def test_backward_frozen_layers_fp32():
    """trainFrom = 2 without embeddings: layers 0-1 and the embeddings get
    exactly zero, the rest match (TestForwardBackwardMatchesPyTorch's frozen
    rule, nn_test.go:139-150)."""
    from decide_amd.train import TrainEngine

    cfg = small_cfg()
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1, seed=1)
    print("case: frozen layers fp32", flush=True)
    _, dl, want = oracle_grads(cfg, w, batch, train_from=2, train_emb=False)
    with TrainEngine(cfg, w, precision="fp32", train_from=2, train_emb=False) as eng:
        eng.forward(batch)
        eng.backward(dl)
        check_grads(eng, want, "fp32", train_from=2, train_emb=False, label="frozen")


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_backward_frozen_layers_small_batch(prec):
    """A training forward of at most 128 tokens (the size at which inference
    splits the residual GEMMs over K): frozen layers 0-1 and trainable layer 2
    give the oracle's gradients (fp32 bar; bf16 against the oracle on the same
    bf16-rounded projection weights at the bf16 bar), and the logits match an
    inference forward of the same batch to fp32 rounding in fp32."""
    from decide_amd import Engine
    from decide_amd.train import TrainEngine

    cfg = small_cfg()
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1, seed=11, specs=[(30, [5, 6], True), (60, [10, 12], True)])
    assert sum(len(s.ids) for s in batch) <= 128
    print(f"case: frozen layers, small batch {prec}", flush=True)
    wref = effective_weights(w, prec)
    _, dl, want = oracle_grads(cfg, wref, batch, train_from=2, train_emb=False)
    with TrainEngine(cfg, w, precision=prec, train_from=2, train_emb=False) as eng:
        got = eng.forward(batch)
        eng.backward(dl)
        check_grads(eng, want, prec, train_from=2, train_emb=False, label="frozen small batch")
    if prec == "fp32":
        with Engine(cfg, w, precision="fp32") as inf:
            ref = inf.forward(batch)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-5 * (1 + np.abs(ref)))


def test_backward_head_only_fp32():
    """trainFrom = Layers: only the final norm and the scorer head get
    gradients; no layer keeps activations (forward.go:226-236)."""
    from decide_amd.train import TrainEngine

    cfg = small_cfg(layers=2)
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1, seed=6)
    print("case: head only fp32", flush=True)
    _, dl, want = oracle_grads(cfg, w, batch, train_from=cfg.layers, train_emb=False)
    with TrainEngine(cfg, w, precision="fp32", train_from=cfg.layers, train_emb=False) as eng:
        eng.forward(batch)
        eng.backward(dl)
        check_grads(eng, want, "fp32", train_from=cfg.layers, train_emb=False, label="head-only")


def test_backward_accumulates_and_zero_grad():
    """Two backward passes add (the kernels are deterministic, so exactly
    2x); dn_zero_grad clears every gradient."""
    from decide_amd.nn import tensor_shapes
    from decide_amd.train import TrainEngine

    cfg = small_cfg(layers=2)
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1, seed=2)
    print("case: accumulate bf16", flush=True)
    _, dl, _ = oracle_grads(cfg, w, batch)
    with TrainEngine(cfg, w, precision="bf16") as eng:
        eng.forward(batch)
        eng.backward(dl)
        once = {n: eng.download(n, "grad") for n in tensor_shapes(cfg)}
        eng.forward(batch)
        eng.backward(dl)
        for n, g in once.items():
            got = eng.download(n, "grad")
            if n == "model.embeddings.tok_embeddings.weight":
                # dTok[id] += dE[t] per token, in token order (backward.go:102-108):
                # a repeated id's second pass adds onto the first pass's sum.
                assert rel_err(got, 2 * g) <= 1e-6, n
            else:
                assert np.array_equal(got, 2 * g), n
        eng.zero_grad()
        assert all(not np.any(eng.download(n, "grad")) for n in once)
        assert eng.grad_sumsq() == 0.0


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_adamw_matches_closed_form_and_oracle(prec):
    """Step 1 from zero moments equals p - (rate*g'/(|g'|+eps) + wd*rate*p)
    with g' = scale*g; grad_sumsq equals the float64 sum of the downloaded
    gradients; two steps equal the oracle's AdamW run on the same
    gradients; after an update the inference forward uses the new weights
    (its logits equal a fresh engine's loaded with them)."""
    from decide_amd.nn import Engine, tensor_shapes
    from decide_amd.train import TrainEngine

    cfg = small_cfg(layers=2)
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1, seed=3)
    print(f"case: adamw {prec}", flush=True)
    _, dl, _ = oracle_grads(cfg, w, batch)
    shapes = tensor_shapes(cfg)
    lr, head_lr, wd, scale = 1e-3, 3e-3, 0.01, 0.5
    with TrainEngine(cfg, w, precision=prec, train_from=1, train_emb=False) as eng:
        eng.forward(batch)
        eng.backward(dl)
        grads = {n: eng.download(n, "grad") for n in shapes}
        trainable = [n for n in shapes if not frozen(n, 1, False)]
        ss = sum(float((grads[n].astype(np.float64) ** 2).sum()) for n in trainable)
        assert abs(eng.grad_sumsq() - ss) <= 1e-12 * ss
        eng.update(lr, head_lr, wd, scale)
        for n, shape in shapes.items():
            p0, p1 = w[n].astype(np.float64), eng.download(n).astype(np.float64)
            if n not in trainable:
                assert np.array_equal(p1, p0), n
                continue
            rate = head_lr if n.startswith("scorer.") else lr
            decay = len(shape) == 2 and n != "model.embeddings.tok_embeddings.weight"
            gs = grads[n].astype(np.float64) * scale
            want = p0 - (rate * gs / (np.abs(gs) + 1e-8) + (wd * rate if decay else 0.0) * p0)
            assert np.allclose(p1, want, rtol=0, atol=2e-6 * max(1.0, float(np.abs(p0).max()))), n
            assert np.allclose(eng.download(n, "m"), 0.1 * gs, rtol=1e-5, atol=1e-12), n
        eng.update(lr, head_lr, wd, scale)  # second step on the same gradients
        # The oracle's AdamW on the device's gradients, two steps.
        om = oracle.OracleModel(cfg, w)
        og = oracle.OracleModel(cfg, grads)
        opt = oracle.OracleAdamW(om, og, weight_decay=wd, train_from=1, train_emb=False)
        opt.update(lr, head_lr, scale)
        opt.update(lr, head_lr, scale)
        for n, shape in shapes.items():
            got = eng.download(n).reshape(-1)
            ref = om.get(n, got.size)
            assert np.max(np.abs(got - ref)) <= 1e-7 * max(1.0, float(np.abs(ref).max())), n
        new_w = {n: eng.download(n) for n in shapes}
        after = eng.infer(batch)
    with Engine(cfg, new_w, precision=prec) as fresh:
        assert np.array_equal(fresh.forward(batch), after)


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_backward_matches_oracle_modernbert_base(prec):
    """ModernBERT-base geometry (22 layers, hidden 768, window 64): a cfg2
    Choice request (112 tokens) and a 300-token plain sequence."""
    from decide_amd import modernbert_base
    from decide_amd.synth import config_batch, pack_request
    from decide_amd.nn import build_sequence, MASK_ID
    from decide_amd.train import TrainEngine

    cfg = modernbert_base()
    w = weights_for(cfg, seed=7, std=0.02)
    rng = np.random.default_rng(9)
    batch = config_batch("cfg2", vocab=cfg.vocab) + [
        build_sequence(pack_request(rng, 260, [20, 20], cfg.vocab), MASK_ID, independent=False)]
    print(f"case: modernbert-base backward {prec}, T={sum(len(s.ids) for s in batch)}", flush=True)
    want_logits, dl, want = oracle_grads(cfg, effective_weights(w, prec), batch)
    with TrainEngine(cfg, w, precision=prec) as eng:
        logits = eng.forward(batch)
        if prec == "fp32":
            assert np.all(np.abs(logits.astype(np.float64) - want_logits) <= 1e-4 * (1 + np.abs(want_logits)))
        eng.backward(dl)
        check_grads(eng, want, prec, label="base")


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_backward_matches_oracle_medium_rows(prec):
    """ModernBERT-base at a trainer-like micro-batch of 4 examples x 384
    tokens (1,536 rows): the medium-M GEMM tiles (64 x 192 for the 768-wide
    fp32 outputs and the GeGLU backward, 128 x 128 stores) against the
    oracle."""
    from decide_amd import modernbert_base
    from decide_amd.nn import MASK_ID, build_sequence
    from decide_amd.synth import pack_request
    from decide_amd.train import TrainEngine

    cfg = modernbert_base()
    w = weights_for(cfg, seed=13, std=0.02)
    rng = np.random.default_rng(14)
    batch = [build_sequence(pack_request(rng, 256, [16] * 8, cfg.vocab), MASK_ID, True) for _ in range(4)]
    print(f"case: modernbert-base backward {prec}, T={sum(len(s.ids) for s in batch)}", flush=True)
    _, dl, want = oracle_grads(cfg, effective_weights(w, prec), batch)
    with TrainEngine(cfg, w, precision=prec) as eng:
        eng.forward(batch)
        eng.backward(dl)
        check_grads(eng, want, prec, label="medium")


def test_backward_full_size_deterministic_and_linear():
    """At the trainer's micro-batch size (10 examples x 384 tokens under the
    4000-token budget, ModernBERT-base, bf16, embeddings trained): a second
    backward of the same forward gives bit-identical gradients (the weight
    gradients run on a second stream, so an unsynchronised buffer would show
    here), and the backward of 2 x dlogits after a fresh forward gives exactly
    twice every gradient (the backward is linear in dlogits and scaling by 2
    commutes with every rounding)."""
    from decide_amd import modernbert_base
    from decide_amd.nn import MASK_ID, build_sequence, tensor_shapes
    from decide_amd.synth import pack_request, random_weights
    from decide_amd.train import TrainEngine

    cfg = modernbert_base()
    w = random_weights(cfg, seed=11)
    rng = np.random.default_rng(12)
    batch = [build_sequence(pack_request(rng, 256, [16] * 8, cfg.vocab), MASK_ID, True) for _ in range(10)]
    R = sum(len(s.mask_pos) for s in batch)
    dl = (rng.standard_normal(R) * 0.1).astype(np.float32)
    print(f"case: full-size backward determinism, T={sum(len(s.ids) for s in batch)}", flush=True)
    names = list(tensor_shapes(cfg))
    with TrainEngine(cfg, w, precision="bf16", train_from=0, train_emb=True) as eng:
        eng.forward(batch)
        eng.backward(dl)
        once = {n: eng.download(n, "grad") for n in names}
        for n, g in once.items():
            assert np.all(np.isfinite(g)) and np.any(g), n
        eng.zero_grad()
        eng.backward(dl)
        for n, g in once.items():
            assert np.array_equal(eng.download(n, "grad"), g), n
        eng.zero_grad()
        eng.forward(batch)
        eng.backward(2 * dl)
        for n, g in once.items():
            assert np.array_equal(eng.download(n, "grad"), 2 * g), n


def test_training_errors():
    """Backward needs a training forward (an inference forward invalidates
    it) and the forward's row count; training must be enabled before bf16
    weights are uploaded."""
    from decide_amd import native
    from decide_amd.nn import Engine
    from decide_amd.train import TrainEngine

    cfg = small_cfg(layers=2)
    w = weights_for(cfg)
    batch = train_batch(cfg.vocab, cfg.vocab - 1)
    R = sum(len(s.mask_pos) for s in batch)
    with TrainEngine(cfg, w, precision="bf16") as eng:
        with pytest.raises(native.InvalidArgument):
            eng.backward(np.zeros(R, np.float32))
        eng.forward(batch)
        with pytest.raises(native.InvalidArgument):
            eng.backward(np.zeros(R + 1, np.float32))
        eng.infer(batch)
        with pytest.raises(native.InvalidArgument):
            eng.backward(np.zeros(R, np.float32))
        eng.forward(batch)
        eng.backward(np.zeros(R, np.float32))
    with Engine(cfg, w, precision="bf16") as eng:
        rc = native.lib.dn_enable_training(eng.handle)
        assert rc == native.DN_INVALID_ARG


def test_training_reduces_loss():
    """Five AdamW steps on one batch lower the trainer's soft cross-entropy
    (internal/train/trainer.go:308-321) in bf16."""
    from decide_amd.train import TrainEngine, soft_cross_entropy

    cfg = small_cfg()
    w = weights_for(cfg, std=0.05)
    batch = train_batch(cfg.vocab, cfg.vocab - 1, seed=4)
    rng = np.random.default_rng(0)
    targets = [np.eye(len(s.mask_pos))[int(rng.integers(0, len(s.mask_pos)))] for s in batch]
    losses = []
    with TrainEngine(cfg, w, precision="bf16") as eng:
        for _ in range(6):
            logits = eng.forward(batch)
            loss, dl = soft_cross_entropy(logits, targets, len(batch))
            losses.append(loss)
            eng.backward(dl)
            gn = eng.grad_norm()
            eng.update(1e-3, 1e-3, 0.01, min(1.0, 1.0 / (gn + 1e-6)))
            eng.zero_grad()
    print("losses", [round(x, 4) for x in losses], flush=True)
    assert losses[-1] < losses[0]
