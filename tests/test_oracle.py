"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker:
against the reference's own PyTorch fixture, against float64 brute force on
the reference GEMM test's shape list, and against closed forms."""
import math

import numpy as np
import pytest

import oracle
from conftest import rel_err, tiny_config, tiny_weights

# internal/blas/gemm_test.go:45
SHAPES = [(1, 1, 1), (6, 16, 8), (7, 17, 9), (13, 33, 300), (100, 250, 257), (5, 800, 64), (200, 5, 512),
          (97, 768, 768), (300, 50, 1)]


def naive(ta, tb, M, N, K, A, lda, B, ldb):
    """gemm_test.go:10-33 in float64."""
    a = (A[: K * lda].reshape(K, lda)[:, :M].T if ta else A[: M * lda].reshape(M, lda)[:, :K]).astype(np.float64)
    b = (B[: N * ldb].reshape(N, ldb)[:, :K].T if tb else B[: K * ldb].reshape(K, ldb)[:, :N]).astype(np.float64)
    return a @ b


@pytest.mark.parametrize("shape", SHAPES)
def test_sgemm_matches_float64(shape):
    """TestSgemm: all transposes x accumulate, tol 1e-3*sqrt(K+1)."""
    rng = np.random.default_rng(3)
    M, N, K = shape
    oracle.set_workers(4)
    for ta in (False, True):
        for tb in (False, True):
            lda = M if ta else K
            ldb = K if tb else N
            A = rng.standard_normal(M * K, dtype=np.float32)
            B = rng.standard_normal(K * N, dtype=np.float32)
            want = naive(ta, tb, M, N, K, A, lda, B, ldb)
            for acc in (False, True):
                C0 = rng.standard_normal(M * N, dtype=np.float32)
                C = C0.copy()
                oracle.sgemm(ta, tb, M, N, K, A, lda, B, ldb, C, N, acc)
                w = want.reshape(-1) + (C0.astype(np.float64) if acc else 0)
                assert np.max(np.abs(C - w)) <= 1e-3 * math.sqrt(K + 1), (shape, ta, tb, acc)
                # The blocked, threaded restatement is bit-identical to the
                # per-element summation order it is derived from.
                Cr = C0.copy()
                oracle.sgemm(ta, tb, M, N, K, A, lda, B, ldb, Cr, N, acc, ref=True)
                assert np.array_equal(C.view(np.uint32), Cr.view(np.uint32)), (shape, ta, tb, acc)


def test_sgemm_leading_dims():
    """TestSgemmLeadingDims: padded lda/ldb/ldc, columns beyond N untouched."""
    rng = np.random.default_rng(4)
    M, N, K = 20, 30, 40
    lda, ldb, ldc = K + 3, N + 5, N + 7
    A = rng.standard_normal(M * lda, dtype=np.float32)
    B = rng.standard_normal(K * ldb, dtype=np.float32)
    C = np.zeros(M * ldc, np.float32)
    oracle.sgemm(False, False, M, N, K, A, lda, B, ldb, C, ldc, False)
    want = naive(False, False, M, N, K, A, lda, B, ldb)
    C2 = C.reshape(M, ldc)
    assert np.max(np.abs(C2[:, :N] - want)) <= 1e-3
    assert np.all(C2[:, N:] == 0)


def test_sgemm_thread_count_invariant():
    """Each C element is owned by one job: any worker count gives the same bits."""
    rng = np.random.default_rng(5)
    M, N, K = 300, 512, 600
    A = rng.standard_normal(M * K, dtype=np.float32)
    B = rng.standard_normal(N * K, dtype=np.float32)
    outs = []
    for w in (1, 3, 8):
        C = np.zeros(M * N, np.float32)
        oracle.sgemm(False, True, M, N, K, A, K, B, K, C, N, False, workers=w)
        outs.append(C)
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def _tiny(tiny_ref):
    from decide_amd.nn import build_sequence

    tensors, meta = tiny_ref
    cfg = tiny_config(meta)
    model = oracle.OracleModel(cfg, tiny_weights(tensors, cfg))
    batch = [build_sequence(s["ids"], meta["mask_id"], s["independent"]) for s in meta["seqs"]]
    return tensors, meta, cfg, model, batch


def test_forward_matches_pytorch_fixture(tiny_ref):
    """TestForwardBackwardMatchesPyTorch (nn_test.go:105-126), forward half,
    plus the fixture's debug activations of sequence 0."""
    tensors, meta, cfg, model, batch = _tiny(tiny_ref)
    oracle.set_workers(4)
    logits, dbg = model.forward(batch, debug=True)
    assert rel_err(logits, tensors["logits"]) <= 1e-4
    n0 = len(batch[0].ids)
    for l in range(4):  # hidden.0 = emb norm output, hidden.l = output of layer l-1
        assert rel_err(dbg["hs"][l, :n0], tensors[f"hidden.{l}"]) <= 1e-5, l
    assert rel_err(dbg["n1"][1, :n0], tensors["l1.n1"]) <= 1e-5
    assert rel_err(dbg["attn"][1, :n0], tensors["l1.attn"]) <= 1e-5
    # loss (nn_test.go:124-127): mean cross-entropy over the two sequences.
    loss, off = 0.0, 0
    for s, spec in zip(batch, meta["seqs"]):
        k = len(s.mask_pos)
        z = logits[off: off + k].astype(np.float64)
        z = z - z.max()
        loss -= (z[spec["target"]] - np.log(np.exp(z).sum())) / len(batch)
        off += k
    assert abs(loss - float(tensors["loss"][0])) <= 1e-4


def test_forward_independent_of_thread_count(tiny_ref):
    _, _, _, model, batch = _tiny(tiny_ref)
    oracle.set_workers(1)
    a = model.forward(batch)
    oracle.set_workers(8)
    b = model.forward(batch)
    assert np.array_equal(a, b)


def test_order_invariance(tiny_ref):
    """TestOrderInvariance (nn_test.go:164-206): permuting option spans
    permutes the logits, within 1e-5."""
    from decide_amd.nn import build_sequence

    tensors, meta, cfg, model, _ = _tiny(tiny_ref)
    base = list(meta["seqs"][0]["ids"])
    mask = meta["mask_id"]
    starts = [i for i, t in enumerate(base) if t == mask]
    last = len(base) - 1
    spans = [base[s: (starts[k + 1] if k + 1 < len(starts) else last)] for k, s in enumerate(starts)]

    def build(order):
        ids = base[: starts[0]]
        for k in order:
            ids = ids + spans[k]
        return ids + [base[last]]

    orig = model.forward([build_sequence(build([0, 1, 2]), mask, True)])
    perm = [2, 0, 1]
    got = model.forward([build_sequence(build(perm), mask, True)])
    for slot, k in enumerate(perm):
        assert abs(float(got[slot]) - float(orig[k])) <= 1e-5


def test_build_sequence_matches_fixture_layout(tiny_ref):
    """gen_ref.py's make_seq positions/options for the independent sequence."""
    _, meta, _, _, batch = _tiny(tiny_ref)
    s = batch[0]
    ids = meta["seqs"][0]["ids"]
    mp = [i for i, t in enumerate(ids) if t == meta["mask_id"]]
    assert list(s.mask_pos) == mp
    last = len(ids) - 1
    for k, st in enumerate(mp):
        e = mp[k + 1] if k + 1 < len(mp) else last
        assert all(s.opt[i] == k and s.pos[i] == mp[0] + i - st for i in range(st, e))
    assert s.opt[last] == -1 and s.pos[last] == last and all(s.opt[i] == -1 for i in range(mp[0]))
    plain = batch[1]
    assert plain.opt is None and list(plain.pos) == list(range(len(plain.ids)))
    # The oracle's own BuildSequence agrees with the library's.
    p2, o2, m2 = oracle.build_sequence(ids, meta["mask_id"], True)
    assert np.array_equal(p2, s.pos) and np.array_equal(o2, s.opt) and np.array_equal(m2, s.mask_pos)


def test_layer_norm_closed_forms():
    x = np.full((3, 64), 2.5, np.float32)
    w = np.linspace(0.5, 2.0, 64).astype(np.float32)
    b = np.linspace(-1, 1, 64).astype(np.float32)
    assert np.all(oracle.layer_norm(x, w, None, 1e-5) == 0)
    assert np.array_equal(oracle.layer_norm(x, w, b, 1e-5), np.tile(b, (3, 1)))
    rng = np.random.default_rng(0)
    y = oracle.layer_norm(rng.standard_normal((5, 768)).astype(np.float32), np.ones(768, np.float32), None, 1e-5)
    assert np.allclose(y.mean(1), 0, atol=1e-6) and np.allclose(y.var(1), 1, rtol=1e-4)


def test_rope_closed_forms():
    cs, sn = oracle.rope_tables(np.array([0, 1, 7, 300], np.int32), 64, 10000.0)
    assert np.all(cs[:32] == 1) and np.all(sn[:32] == 0)  # position 0 is the identity
    # frequency 0 is 1/theta^0 = 1: angle == position
    assert cs[32] == np.float32(math.cos(1.0)) and sn[64] == np.float32(math.sin(7.0))
    T, H, heads, D = 4, 128, 2, 64
    rng = np.random.default_rng(1)
    qkv = rng.standard_normal(T * 3 * H).astype(np.float32)
    before = qkv.reshape(T, 3 * H).copy()
    oracle.apply_rope(qkv, T, H, heads, D, cs, sn)
    after = qkv.reshape(T, 3 * H)
    assert np.array_equal(after[0], before[0])
    assert np.array_equal(after[:, 2 * H:], before[:, 2 * H:])  # v untouched
    for hd in range(heads):
        for off in (hd * D, H + hd * D):
            n0 = before[:, off: off + 32] ** 2 + before[:, off + 32: off + 64] ** 2
            n1 = after[:, off: off + 32] ** 2 + after[:, off + 32: off + 64] ** 2
            assert np.allclose(n0, n1, rtol=1e-5)


def test_gelu_closed_forms():
    assert oracle.gelu(0.0) == 0.0
    assert oracle.gelu(10.0) == np.float32(10.0)
    assert abs(oracle.gelu(-10.0)) < 1e-20
    assert abs(oracle.gelu(1.0) - 0.8413447460685429) < 1e-6  # 1 * Phi(1)


def test_softmax_masked_closed_forms():
    rng = np.random.default_rng(2)
    n = 9
    P = rng.standard_normal(n * n).astype(np.float32)
    mask = (rng.random(n * n) < 0.5).astype(np.uint8)
    mask[:: n + 1] = 1  # every row keeps itself
    oracle.softmax_masked(P, n, 0.125, mask)
    P = P.reshape(n, n)
    assert np.all(P[mask.reshape(n, n) == 0] == 0)
    assert np.allclose(P.sum(1), 1, atol=1e-6)


def test_answer_post_processing():
    """TestMarginConfidence (types_test.go:206-216), argmax ties, RoundToEven."""
    assert oracle.margin_confidence([1.0]) == 1
    assert oracle.margin_confidence([0.5, 0.5]) == 0
    assert oracle.margin_confidence([0.9, 0.05, 0.05]) == 0.85
    assert oracle.argmax([1.0, 3.0, 3.0]) == 1
    assert oracle.round_even(0.125, 2) == 0.12 and oracle.round_even(0.135, 2) == 0.14
    p = oracle.calibrated([1.0, 2.0, 3.0], 2.0)
    e = np.exp(np.array([0.5, 1.0, 1.5]) - 1.5)
    assert np.allclose(p, e / e.sum(), rtol=0, atol=1e-15)
    assert np.allclose(oracle.calibrated([1.0, 2.0], 0.0), oracle.calibrated([1e4, 2e4], 1.0))
