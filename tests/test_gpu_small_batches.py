"""Small batches at ModernBERT-base size against the CPU oracle, with the
total token count T swept across the small-M GEMM's tile rules (every
projection runs the whole-K kernel up to 128 rows: 32-row tiles while the
grid fits one workgroup per CU, 64-row tiles past it; Wi + GeGLU on 32- or
64-column tiles by the same rule), the split counts of the residual GEMMs
(Wo / MlpWo split over K into 2 to 6 parts that the next LayerNorm sums,
fewer parts as T grows) and the forward prologue's 32-token chunks (ragged
sequences, one to three per batch, independent and plain).

Bars as in test_gpu_forward: fp32 max |dp| <= 1e-5 and logits within
1e-4 * (1 + |logit|); bf16 and fp16 max |dp| <= 2e-3; argmax agreement
(16-bit modes: on every request whose oracle top-two probabilities are more
than 4e-3 apart)."""
import numpy as np
import pytest

import oracle
from test_gpu_forward import WORKERS, compare

pytestmark = pytest.mark.gpu

# T values on both sides of the boundaries: 32 / 64 / 96 / 128 rows, and
# the grid sizes (N / 32) * ceil(T / 32) around 256 workgroups for N = 2304.
TOTALS = [9, 31, 33, 63, 64, 65, 96, 97, 112, 127, 128]


def batch_with_total(total, vocab, rng):
    """One to three packed requests whose lengths add up to `total`."""
    from decide_amd.nn import build_sequence
    from decide_amd.synth import MASK_ID, pack_request

    nseq = int(rng.integers(1, min(3, total // 9) + 1))
    # each sequence at least 9 tokens, the rest spread at random
    lens = 9 + rng.multinomial(total - 9 * nseq, [1.0 / nseq] * nseq)
    batch = []
    for i, n in enumerate(lens):
        k = int(rng.integers(1, min(4, (n - 3) // 2) + 1))  # options, each at least 2 tokens
        premise = int(rng.integers(3, n - 2 * k + 1))  # [CLS] ... [SEP], at least 3 tokens
        rest = n - premise
        opt = [2] * k
        for j in range(rest - 2 * k):
            opt[j % k] += 1
        ids = pack_request(rng, premise, opt, vocab)
        assert len(ids) == n
        batch.append(build_sequence(ids, MASK_ID, independent=bool(i % 2 == 0)))
    return batch


@pytest.fixture(scope="module")
def base_small():
    from decide_amd import Engine, NoGPUError, modernbert_base
    from decide_amd.synth import random_weights

    cfg = modernbert_base()
    w = random_weights(cfg, seed=3)
    try:
        engs = {p: Engine(cfg, w, precision=p) for p in ("fp32", "bf16", "fp16")}
    except NoGPUError:
        pytest.skip("no GPU")
    yield cfg, oracle.OracleModel(cfg, w), engs
    for e in engs.values():
        e.close()


@pytest.mark.parametrize("total", TOTALS)
def test_small_batch_matches_oracle(base_small, total):
    cfg, orc, engs = base_small
    rng = np.random.default_rng(1000 + total)
    batch = batch_with_total(total, cfg.vocab, rng)
    assert sum(len(s.ids) for s in batch) == total
    oracle.set_workers(WORKERS)
    want = orc.forward(batch)
    for prec in ("fp32", "bf16", "fp16"):
        compare(engs[prec].forward(batch), want, batch, prec)


@pytest.mark.parametrize("prec", ["bf16", "fp16"])
def test_small_m_operand_paths_agree(base_small, prec):
    """dn_set_small_m_loads: the small-M GEMM's two operand paths (whole rows
    through LDS by global->LDS DMA, the default; fragments straight into
    registers) feed the MFMAs the same operands in the same order, so every
    batch size gives bit-identical logits."""
    cfg, _, engs = base_small
    eng = engs[prec]
    rng = np.random.default_rng(77)
    try:
        for total in TOTALS:
            batch = batch_with_total(total, cfg.vocab, rng)
            eng.set_small_m_loads(1)
            lds = eng.forward(batch)
            eng.set_small_m_loads(0)
            regs = eng.forward(batch)
            assert np.array_equal(lds, regs), (total, float(np.max(np.abs(lds - regs))))
    finally:
        eng.set_small_m_loads(1)
