"""The reference's own PyTorch fixture on the GPU, and other geometries the
MFMA kernels do not tile.

tests/golden/tiny_ref.safetensors (the reference's
internal/nn/testdata/tiny_ref.safetensors) is hidden 32, 4 heads of 8,
intermediate 48: the library runs it on its any-shape GEMM and attention
kernels. Bars:
- fp32 mode against the fixture's PyTorch logits: relErr <= 1e-4, the bar of
  TestForwardBackwardMatchesPyTorch (nn_test.go:105-126); against the oracle
  at max |dlogit| <= 1e-5 (1 + |logit|);
- bf16 mode (bf16 GEMM operands) against the oracle given the same
  bf16-rounded projection weights: option probabilities within 2e-3, as the
  forward tests.
A second geometry (hidden 96, 6 heads of 16, intermediate 80, a window that
matters) checks the same path against the oracle with ragged sequences."""
import numpy as np
import pytest

import oracle
from conftest import rel_err, tiny_config, tiny_weights

pytestmark = pytest.mark.gpu


def bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(np.shape(a))


PROJ = ("attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight")


def probs(logits, batch):
    out, off = [], 0
    for s in batch:
        k = len(s.mask_pos)
        z = np.asarray(logits[off:off + k], np.float64)
        e = np.exp(z - z.max())
        out.append(e / e.sum())
        off += k
    return np.concatenate(out)


def engine(cfg, w, prec):
    from decide_amd import Engine, NoGPUError

    try:
        return Engine(cfg, w, precision=prec)
    except NoGPUError:
        pytest.skip("no GPU")


def fixture_batch(meta):
    from decide_amd.nn import build_sequence

    return [build_sequence(s["ids"], meta["mask_id"], s["independent"]) for s in meta["seqs"]]


def test_reference_fixture_fp32(tiny_ref):
    tensors, meta = tiny_ref
    cfg = tiny_config(meta)
    w = tiny_weights(tensors, cfg)
    batch = fixture_batch(meta)
    print(f"case: tiny_ref fp32, {len(batch)} sequences", flush=True)
    with engine(cfg, w, "fp32") as eng:
        got = eng.forward(batch)
        alone = np.concatenate([eng.forward([s]) for s in batch])
    err = rel_err(got, tensors["logits"])
    print(f"relErr against the PyTorch logits {err:.3g}")
    assert err <= 1e-4
    # and the fixture's loss (nn_test.go:124-127): mean cross-entropy over the sequences
    loss, off = 0.0, 0
    for s, spec in zip(batch, meta["seqs"]):
        k = len(s.mask_pos)
        z = got[off: off + k].astype(np.float64)
        z = z - z.max()
        loss -= (z[spec["target"]] - np.log(np.exp(z).sum())) / len(batch)
        off += k
    assert abs(loss - float(tensors["loss"][0])) <= 1e-4
    oracle.set_workers(4)
    want = oracle.OracleModel(cfg, w).forward(batch)
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * (1 + np.abs(want)))
    assert np.all(np.abs(alone.astype(np.float64) - got) <= 1e-5 * (1 + np.abs(got)))


def test_reference_fixture_bf16(tiny_ref):
    tensors, meta = tiny_ref
    cfg = tiny_config(meta)
    w = tiny_weights(tensors, cfg)
    batch = fixture_batch(meta)
    print(f"case: tiny_ref bf16, {len(batch)} sequences", flush=True)
    with engine(cfg, w, "bf16") as eng:
        got = eng.forward(batch)
    oracle.set_workers(4)
    wb = {n: (bf16_round(a) if n.endswith(PROJ) else a) for n, a in w.items()}
    want = oracle.OracleModel(cfg, wb).forward(batch)
    dp = float(np.max(np.abs(probs(got, batch) - probs(want, batch))))
    print(f"bf16 max |dp| {dp:.3g}, relErr against PyTorch {rel_err(got, tensors['logits']):.3g}")
    assert dp <= 2e-3


@pytest.mark.parametrize("prec", ["fp32", "bf16", "fp16"])
def test_generic_geometry_matches_oracle(prec):
    """hidden 96, 6 heads of 16, intermediate 80, half window 8, global and
    local layers; an independent-options sequence, a plain one and a short
    one in one batch."""
    from decide_amd.nn import Config, build_sequence
    from decide_amd.synth import random_weights

    cfg = Config(hidden=96, intermediate=80, heads=6, layers=3, vocab=300, half_window=8,
                 layer_types=["full_attention", "sliding_attention", "sliding_attention"])
    w = random_weights(cfg, seed=7, std=0.05)
    rng = np.random.default_rng(2)
    batch = []
    for prem, opts, indep in [(40, [4, 5, 6], True), (70, [9, 9], False), (3, [2, 1], True)]:
        ids = [1] + list(rng.integers(3, 299, size=prem)) + [2]
        for ln in opts:
            ids += [299] + list(rng.integers(3, 299, size=ln - 1))
        batch.append(build_sequence(np.array(ids + [2], np.int32), 299, independent=indep))
    print(f"case: generic geometry {prec}", flush=True)
    with engine(cfg, w, prec) as eng:
        got = eng.forward(batch)
    oracle.set_workers(4)
    rnd = {"fp32": None, "bf16": bf16_round, "fp16": lambda a: np.asarray(a, np.float16).astype(np.float32)}[prec]
    wb = w if rnd is None else {n: (rnd(a) if n.endswith(PROJ) else a) for n, a in w.items()}
    want = oracle.OracleModel(cfg, wb).forward(batch)
    if prec == "fp32":
        assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * (1 + np.abs(want)))
    else:
        assert float(np.max(np.abs(probs(got, batch) - probs(want, batch)))) <= 2e-3


def test_generic_geometry_refuses_training(tiny_ref):
    """Training stays on the MFMA geometry: dn_enable_training reports
    DN_UNSUPPORTED for the fixture's config."""
    from decide_amd import NoGPUError, Unsupported
    from decide_amd.train import TrainEngine

    tensors, meta = tiny_ref
    cfg = tiny_config(meta)
    with pytest.raises((Unsupported, NoGPUError)) as ei:
        TrainEngine(cfg, tiny_weights(tensors, cfg), precision="fp32")
    if isinstance(ei.value, NoGPUError):
        pytest.skip("no GPU")
