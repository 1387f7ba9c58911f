"""Forward parity on the GPU: libdecide_hip.so against the CPU oracle on
identical seeded weights and token ids.

Bars: per-option probabilities (softmax over each
question's logits, T = 1) within max |dp| <= 1e-5 in the fp32 validation
mode and <= 2e-3 in the 16-bit modes (bf16, fp16), argmax agreement; logits
are also compared directly (fp32: |dlogit| <= 1e-4 * (1 + |logit|))."""
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

WORKERS = max(1, min(16, os.cpu_count() or 1))


def probs_per_seq(logits, batch):
    out, off = [], 0
    for s in batch:
        k = len(s.mask_pos)
        z = np.asarray(logits[off: off + k], np.float64)
        e = np.exp(z - z.max())
        out.append(e / e.sum())
        off += k
    return out


def compare(got, want, batch, prec, bf16_dp=2e-3):
    """fp32: every argmax and the 1e-5 bars. 16-bit modes: max |dp| <=
    bf16_dp and the argmax of every request whose oracle top-two
    probabilities are more than 2 x bf16_dp apart (a near-tie inside the
    tolerance may order either way; the agreement rate over many requests is
    test_argmax_agreement_1000_requests' bar)."""
    pg, pw = probs_per_seq(got, batch), probs_per_seq(want, batch)
    dp = max(float(np.max(np.abs(a - b))) for a, b in zip(pg, pw))
    flips = [i for i, (a, b) in enumerate(zip(pg, pw)) if np.argmax(a) != np.argmax(b)]
    agree = 1.0 - len(flips) / len(pw)
    dl = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    print(f"{prec}: max|dp| {dp:.3g} max|dlogit| {dl:.3g} argmax agree {agree:.4f} "
          f"(logit range {float(np.min(want)):.4g}..{float(np.max(want)):.4g})", flush=True)
    assert np.all(np.isfinite(got))
    if prec == "fp32":
        assert dp <= 1e-5
        assert np.all(np.abs(np.asarray(got, np.float64) - want) <= 1e-4 * (1 + np.abs(want)))
        assert agree == 1.0
    else:
        assert dp <= bf16_dp
        for i in flips:
            top2 = np.sort(pw[i])[-2:]
            assert top2[1] - top2[0] <= 2 * bf16_dp, (i, top2)


# ---------------------------------------------------------------- small geometry
def small_cfg():
    from decide_amd.nn import Config

    return Config(hidden=256, intermediate=384, heads=4, layers=4, vocab=300, half_window=4,
                  layer_types=["full_attention", "sliding_attention", "sliding_attention", "full_attention"])


def ragged_batch(vocab, mask_id, seed=0):
    """Lengths straddling the 32/64/128 tile edges; independent and plain
    sequences mixed; a one-token sequence; options of length 1."""
    from decide_amd.nn import build_sequence

    rng = np.random.default_rng(seed)
    out = []
    specs = [(1, []), (9, [1, 5]), (30, [4, 3]), (33, [16, 15]), (64, [8] * 3), (65, [20, 1, 7]),
             (127, [40, 30]), (128, [64, 64]), (129, [10] * 6), (200, [30, 30, 30])]
    for i, (prem, opts) in enumerate(specs):
        ids = list(rng.integers(2, mask_id, size=prem))
        for ln in opts:
            ids += [mask_id] + list(rng.integers(2, mask_id, size=ln - 1))
        if not opts:
            ids = [mask_id]
        else:
            ids.append(1)
        out.append(build_sequence(np.array(ids, np.int32), mask_id, independent=(i % 3 != 2)))
    return out


@pytest.fixture(scope="module")
def small():
    from decide_amd.synth import random_weights

    cfg = small_cfg()
    w = random_weights(cfg, seed=5, std=0.05)
    return cfg, w, oracle.OracleModel(cfg, w)


@pytest.mark.parametrize("prec", ["fp32", "bf16", "fp16"])
def test_small_geometry_ragged(small, prec):
    from decide_amd import Engine, NoGPUError

    cfg, w, orc = small
    batch = ragged_batch(cfg.vocab, mask_id=cfg.vocab - 1)
    oracle.set_workers(WORKERS)
    want = orc.forward(batch)
    try:
        eng = Engine(cfg, w, precision=prec)
    except NoGPUError:
        pytest.skip("no GPU")
    with eng:
        got = eng.forward(batch)
        # This geometry uses std 0.05 weights (logits spread several times the
        # N(0,0.02) base configs'), which amplifies bf16 operand rounding; its
        # bf16 bar is 1e-2. The fp32 run holds the 1e-5 bar on the same batch.
        compare(got, want, batch, prec, bf16_dp=1e-2)
        # One sequence at a time: up to 128 tokens run the split-K small-M
        # GEMM (another fp32 summation order than the batch's tiles). fp32
        # still gives the batch's logits to 1e-5; bf16 rounds the activations
        # after each GEMM, so each single-sequence run is held to the oracle
        # bar instead.
        off = 0
        for s in batch:
            one = eng.forward([s])
            k = len(s.mask_pos)
            if prec == "fp32":
                assert np.allclose(one, got[off: off + k], rtol=1e-5, atol=1e-6)
            else:
                compare(one, want[off: off + k], [s], prec, bf16_dp=1e-2)
            off += k


def random_layout_batch(vocab, mask_id, seed):
    """A seeded random batch: 1-24 sequences of 1-250 premise tokens and 0-6
    options of 1-40 tokens, plain or independent; a few thousand tokens."""
    from decide_amd.nn import build_sequence

    rng = np.random.default_rng(1000 + seed)
    out = []
    for _ in range(int(rng.integers(1, 25))):
        ids = list(rng.integers(2, mask_id, size=int(rng.integers(1, 251))))
        nopt = int(rng.integers(0, 7))
        for _ in range(nopt):
            ln = int(rng.integers(1, 41))
            ids += [mask_id] + list(rng.integers(2, mask_id, size=ln - 1))
        if nopt == 0:
            ids.append(mask_id)  # every sequence scores at least one row
        ids.append(1)
        out.append(build_sequence(np.array(ids, np.int32), mask_id, independent=bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_random_layouts_match_oracle(small, prec):
    """Seeded random batch layouts (ragged lengths, option counts and
    independence mixed) against the oracle, through each orchestration path
    of the forward: one stream, the two-stream split (threshold lowered so
    that the larger batches take it) and the option-row last layer (forced
    on). fp32 holds the 1e-5 bar on every run; bf16 the small geometry's
    1e-2 bar (its std 0.05 weights, as test_small_geometry_ragged)."""
    from decide_amd import Engine, NoGPUError

    cfg, w, orc = small
    oracle.set_workers(WORKERS)
    try:
        eng = Engine(cfg, w, precision=prec)
    except NoGPUError:
        pytest.skip("no GPU")
    with eng:
        for seed in range(6):
            batch = random_layout_batch(cfg.vocab, cfg.vocab - 1, seed)
            want = orc.forward(batch)
            ntok = sum(len(s.ids) for s in batch)
            for split, tail in ((0, 0), (2048, 0), (0, 1), (2048, 1)):
                eng.set_stream_split(split)
                eng.set_row_tail(tail)
                got = eng.forward(batch)
                print(f"seed {seed}: {len(batch)} sequences, {ntok} tokens, split {split} tail {tail}", flush=True)
                compare(got, want, batch, prec, bf16_dp=1e-2)
        eng.set_stream_split(8192)
        eng.set_row_tail(2048)


# ---------------------------------------------------------------- ModernBERT-base
@pytest.fixture(scope="module")
def base():
    from decide_amd import modernbert_base
    from decide_amd.synth import random_weights

    cfg = modernbert_base()
    w = random_weights(cfg, seed=0)
    return cfg, w, oracle.OracleModel(cfg, w)


@pytest.fixture(scope="module")
def engines(base):
    from decide_amd import Engine, NoGPUError

    cfg, w, _ = base
    try:
        e = {p: Engine(cfg, w, precision=p) for p in ("fp32", "bf16", "fp16")}
    except NoGPUError:
        pytest.skip("no GPU")
    yield e
    for x in e.values():
        x.close()


@pytest.mark.parametrize("name,nseq", [("cfg2", None), ("cfg5", None), ("cfg3", 2), ("cfg4", 1)])
@pytest.mark.parametrize("prec", ["fp32", "bf16", "fp16"])
def test_base_config_matches_oracle(base, engines, name, nseq, prec):
    from decide_amd.synth import config_batch

    cfg, _, orc = base
    batch = config_batch(name, vocab=cfg.vocab, nseq=nseq)
    oracle.set_workers(WORKERS)
    want = orc.forward(batch)
    got = engines[prec].forward(batch)
    compare(got, want, batch, prec)


def test_cfg3_full_batch_properties(base, engines):
    """Full cfg3 (64 x 512, the bench workload). Each sequence's logits do not
    depend on the rest of the batch: bit-for-bit up to fp32 rounding in the
    fp32 mode (|d| <= 1e-4 * (1 + |logit|)); in bf16 the full batch and the
    single-sequence runs (different GEMM tile configs, so different operand
    rounding flips) both stay within the bf16 bar of the oracle. Permuting a
    sequence's options permutes its logits."""
    from decide_amd.nn import build_sequence
    from decide_amd.synth import config_batch

    cfg, _, orc = base
    batch = config_batch("cfg3", vocab=cfg.vocab)
    full = {p: engines[p].forward(batch) for p in ("fp32", "bf16", "fp16")}
    for p in full:
        assert full[p].shape == (512,) and np.all(np.isfinite(full[p]))
    oracle.set_workers(WORKERS)
    for i in (0, 37, 63):
        want = orc.forward([batch[i]])
        one32 = engines["fp32"].forward([batch[i]])
        assert np.all(np.abs(one32 - full["fp32"][8 * i: 8 * i + 8]) <= 1e-4 * (1 + np.abs(one32)))
        compare(full["fp32"][8 * i: 8 * i + 8], want, [batch[i]], "fp32")
        for p in ("bf16", "fp16"):
            compare(full[p][8 * i: 8 * i + 8], want, [batch[i]], p)
            compare(engines[p].forward([batch[i]]), want, [batch[i]], p)
    s = batch[5]
    ids = s.ids.copy()
    starts = list(s.mask_pos)
    last = len(ids) - 1
    spans = [ids[a: (starts[k + 1] if k + 1 < len(starts) else last)] for k, a in enumerate(starts)]
    perm = [3, 7, 0, 1, 6, 2, 5, 4]
    pids = np.concatenate([ids[: starts[0]]] + [spans[k] for k in perm] + [ids[last:]]).astype(np.int32)
    # TestOrderInvariance's 1e-5 in fp32; the 16-bit bar in bf16 and fp16.
    for p, tol in (("fp32", 1e-5), ("bf16", 2e-3), ("fp16", 2e-3)):
        base_one = engines[p].forward([s])
        got = engines[p].forward([build_sequence(pids, 50284, True)])
        for slot, k in enumerate(perm):
            assert abs(float(got[slot]) - float(base_one[k])) <= tol, (p, slot, k)


def test_forward_device_matches_host_entry(base, engines):
    import torch

    from decide_amd.nn import flatten, row_tokens
    from decide_amd.synth import config_batch

    eng = engines["bf16"]
    batch = config_batch("cfg3", vocab=base[0].vocab, nseq=3)
    host = eng.forward(batch)
    seq_len, ids, pos, opt, nmask, _ = flatten(batch)
    d = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=ids, pos=pos, opt=opt, rt=row_tokens(batch)).items()}
    out = torch.zeros(len(host), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    eng.forward_device(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(), len(host),
                       d["rt"].data_ptr(), out.data_ptr())
    eng.check_device_errors()
    assert np.array_equal(out.cpu().numpy(), host)


def test_forward_validation_errors(base, engines):
    """Model.Forward's input validation (forward.go:145-150, 181-183, 192-196)."""
    from decide_amd import InvalidArgument
    from decide_amd.nn import Sequence

    eng = engines["bf16"]
    good = Sequence(ids=np.array([50281, 7, 50284, 9, 50282], np.int32), pos=np.arange(5, dtype=np.int32),
                    opt=None, mask_pos=np.array([2], np.int32))
    assert eng.forward([good]).shape == (1,)
    cases = [
        (Sequence(ids=np.zeros(0, np.int32), pos=np.zeros(0, np.int32), opt=None, mask_pos=np.array([0], np.int32)),
         "nn: malformed sequence 0"),
        (Sequence(ids=good.ids, pos=good.pos, opt=None, mask_pos=np.zeros(0, np.int32)),
         "nn: sequence 0 has no options"),
        (Sequence(ids=good.ids, pos=good.pos, opt=None, mask_pos=np.array([5], np.int32)),
         "nn: sequence 0 mask position 5 out of range"),
        (Sequence(ids=np.array([50281, 50368, 50284], np.int32), pos=np.arange(3, dtype=np.int32), opt=None,
                  mask_pos=np.array([2], np.int32)), "nn: token id 50368 out of range"),
    ]
    for seq, msg in cases:
        with pytest.raises(InvalidArgument) as ei:
            eng.forward([good, seq] if "sequence 0" not in msg else [seq])
        assert ei.value.message == msg
    assert np.isfinite(eng.forward([good])).all()  # the context stays usable


def test_forward_device_position_range_flagged(base, engines):
    """The device-resident entry point cannot validate positions on the host:
    a position past the RoPE tables' range (65535) is flagged by the kernels
    and reported by dn_check_device_errors as unsupported; the context stays
    usable and the next valid batch is correct."""
    import torch
    from decide_amd import Unsupported
    from decide_amd.nn import Sequence, flatten, row_tokens

    eng = engines["bf16"]
    good = Sequence(ids=np.array([50281, 7, 50284, 9, 50282], np.int32), pos=np.arange(5, dtype=np.int32),
                    opt=None, mask_pos=np.array([2], np.int32))
    want = eng.forward([good])
    bad_pos = np.array([0, 1, 70000, 3, 4], np.int32)
    for pos in (bad_pos, good.pos):
        seq_len, ids, _, _, _, _ = flatten([good])
        opt = np.full(len(ids), -1, np.int32)
        d = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=ids, pos=pos, opt=opt, rt=row_tokens([good])).items()}
        out = torch.zeros(1, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        eng.forward_device(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(), 1,
                           d["rt"].data_ptr(), out.data_ptr())
        if pos is bad_pos:
            with pytest.raises(Unsupported):
                eng.check_device_errors()
        else:
            eng.check_device_errors()
            assert np.array_equal(out.cpu().numpy(), want)


def test_option_id_limit(base, engines):
    """Option ids are packed as ((opt + 1) << 16) | pos in a signed 32-bit
    word, so 32766 is the largest id either entry point takes. dn_forward and
    dn_forward_device both accept it (and agree bit for bit); 32767 is refused
    by dn_forward's host check and flagged by dn_forward_device's kernels."""
    import torch
    from decide_amd import Unsupported
    from decide_amd.nn import Sequence, flatten, row_tokens

    eng = engines["bf16"]
    ids = np.array([50281, 7, 50284, 9, 50282], np.int32)
    for oid in (32766, 32767):
        opt = np.array([-1, oid, -1, oid, -1], np.int32)
        seq = Sequence(ids=ids, pos=np.arange(5, dtype=np.int32), opt=opt, mask_pos=np.array([2], np.int32))
        seq_len, fids, fpos, fopt, _, _ = flatten([seq])
        d = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=fids, pos=fpos, opt=fopt,
                                                              rt=row_tokens([seq])).items()}
        out = torch.zeros(1, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        eng.forward_device(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(), 1,
                           d["rt"].data_ptr(), out.data_ptr())
        if oid == 32766:
            host = eng.forward([seq])
            eng.check_device_errors()
            assert np.isfinite(host).all() and np.array_equal(out.cpu().numpy(), host)
        else:
            with pytest.raises(Unsupported) as ei:
                eng.forward([seq])
            assert "option id 32767 outside [-1, 32766]" in ei.value.message
            with pytest.raises(Unsupported):
                eng.check_device_errors()


def test_max_length_sequence(base, engines):
    """The longest sequence this build accepts (8192 tokens, the reference's
    Local limit: 8000-token premise + 4 options x 48) against the oracle in
    both modes; one token more is refused as unsupported."""
    from decide_amd import Unsupported
    from decide_amd.nn import build_sequence
    from decide_amd.synth import pack_request

    cfg, _, orc = base
    rng = np.random.default_rng(8192)
    ids = pack_request(rng, 8000, [48] * 4, cfg.vocab)
    assert len(ids) == 8192
    batch = [build_sequence(ids, 50284, True)]
    oracle.set_workers(WORKERS)
    want = orc.forward(batch)
    for prec in ("fp32", "bf16", "fp16"):
        compare(engines[prec].forward(batch), want, batch, prec)
    long_ids = pack_request(rng, 8001, [48] * 4, cfg.vocab)
    with pytest.raises(Unsupported):
        engines["bf16"].forward([build_sequence(long_ids, 50284, True)])


def _question_probs(logits, groups_per_seq):
    """Softmax (T = 1) within each question's logits: groups_per_seq[i] lists
    (first, K) of sequence i's questions, relative to that sequence."""
    out, off = [], 0
    for groups in groups_per_seq:
        for first, k in groups:
            z = np.asarray(logits[off + first: off + first + k], np.float64)
            e = np.exp(z - z.max())
            out.append(e / e.sum())
        off += sum(k for _, k in groups)
    return out


def test_cfg4_full_batch(base, engines):
    """cfg4 at its configured batch (8 x 2816 tokens, 84 options per
    sequence in 24 questions): two sequences against the oracle, per question,
    in both modes; each sequence's logits do not depend on the rest of the
    batch (fp32: to 1e-4 * (1 + |logit|) against the sequence run alone; bf16:
    the full-batch and single-sequence runs both within the bf16 bar)."""
    from decide_amd.synth import cfg4_question_groups, config_batch

    cfg, _, orc = base
    batch = config_batch("cfg4", vocab=cfg.vocab)
    assert len(batch) == 8 and all(len(s.ids) == 2816 and len(s.mask_pos) == 84 for s in batch)
    groups = [(first, k) for _, first, k in cfg4_question_groups()]
    full = {p: engines[p].forward(batch) for p in ("fp32", "bf16", "fp16")}
    for p in full:
        assert full[p].shape == (8 * 84,) and np.all(np.isfinite(full[p]))
    oracle.set_workers(WORKERS)
    for i in (0, 5):
        want = orc.forward([batch[i]])
        pw = _question_probs(want, [groups])
        for p, bar in (("fp32", 1e-5), ("bf16", 2e-3), ("fp16", 2e-3)):
            part = full[p][84 * i: 84 * i + 84]
            one = engines[p].forward([batch[i]])
            for got in (part, one):
                pg = _question_probs(got, [groups])
                dp = max(float(np.max(np.abs(a - b))) for a, b in zip(pg, pw))
                agree = np.mean([int(np.argmax(a) == np.argmax(b)) for a, b in zip(pg, pw)])
                print(f"cfg4 seq {i} {p}: max|dp| {dp:.3g}, argmax agree {agree:.3f}", flush=True)
                assert dp <= bar
                if p == "fp32":
                    assert agree == 1.0
            if p == "fp32":
                assert np.all(np.abs(one - part) <= 1e-4 * (1 + np.abs(one)))


def test_ln_fold_matches_layernorm_kernels(base, engines):
    """dn_set_ln_fold: bf16 forwards of more than 1024 tokens run attn_norm
    and mlp_norm inside the GEMMs around them (the residual GEMM writes the
    norm's operand bf16((x - m) * w) and per-192-column row statistics; QKV
    and Wi apply rstd and the mean through column sums of the weighted
    projection). Against the same forward with the LayerNorm kernels and
    against the oracle, at the bf16 bar, on batches that take each tile
    configuration of the folded GEMMs: cfg3's 64 x 512 tokens (256 x 192
    residual, 256 x 128 QKV / Wi tiles) on one stream and on two, one cfg4
    sequence (2,816 tokens: 64 x 192 and 128 x 128 tiles), 4,097 and 6,001
    tokens (256 x 192 residual, 256 x 128 QKV and 128 x 128 Wi tiles, the last
    256-row tile holding 1 and 113 rows) and 1,025 tokens (the smallest batch
    that folds; at 1,024 the switch changes nothing, bit for bit). The folded logits are not the unfolded ones (the fold ran).
    fp16 folds the same way (1,025 tokens); the fp32 mode does not fold."""
    from decide_amd.nn import build_sequence
    from decide_amd.synth import config_batch, pack_request

    cfg, _, orc = base
    eng = engines["bf16"]
    rng = np.random.default_rng(91)
    b1025 = [build_sequence(pack_request(rng, p, [16] * 8, cfg.vocab), 50284, True) for p in (385, 384)]
    b1024 = [build_sequence(pack_request(rng, 384, [16] * 8, cfg.vocab), 50284, True) for _ in range(2)]
    assert sum(len(s.ids) for s in b1025) == 1025 and sum(len(s.ids) for s in b1024) == 1024
    b4097 = [build_sequence(pack_request(rng, p, [16] * 8, cfg.vocab), 50284, True) for p in [384] * 7 + [385]]
    b6001 = [build_sequence(pack_request(rng, p, [16] * 8, cfg.vocab), 50284, True) for p in [384] * 11 + [241]]
    assert sum(len(s.ids) for s in b4097) == 4097 and sum(len(s.ids) for s in b6001) == 6001
    off1025 = np.concatenate([[0], np.cumsum([len(s.mask_pos) for s in b1025])])
    cfg3 = config_batch("cfg3", vocab=cfg.vocab)
    cfg4 = config_batch("cfg4", vocab=cfg.vocab, nseq=1)
    oracle.set_workers(WORKERS)
    try:
        for name, batch, split, check in (("cfg3 two streams", cfg3, 8192, (0, 37, 63)), ("cfg3 one stream", cfg3, 0, ()),
                                          ("cfg4 x1", cfg4, 8192, (0,)), ("4097 tokens", b4097, 8192, (7,)),
                                          ("6001 tokens", b6001, 8192, (11,)), ("1025 tokens", b1025, 8192, (0, 1))):
            eng.set_stream_split(split)
            eng.set_ln_fold(False)
            plain = eng.forward(batch)
            eng.set_ln_fold(True)
            folded = eng.forward(batch)
            d = np.abs(folded.astype(np.float64) - plain)
            print(f"ln fold, {name}: max |dlogit| folded vs LayerNorm kernels {float(d.max()):.3g}", flush=True)
            assert not np.array_equal(folded, plain), name
            compare(folded, plain.astype(np.float64), batch, "bf16")
            off = np.concatenate([[0], np.cumsum([len(s.mask_pos) for s in batch])])
            for i in check:
                want = orc.forward([batch[i]])
                compare(folded[off[i]: off[i + 1]], want, [batch[i]], "bf16")
        eng.set_ln_fold(False)
        plain = eng.forward(b1024)
        eng.set_ln_fold(True)
        assert np.array_equal(eng.forward(b1024), plain)
        # fp16 folds as bf16 does (checked at the 16-bit bar against its
        # LayerNorm kernels and the oracle); fp32 does not fold.
        for p in ("fp16", "fp32"):
            engines[p].set_ln_fold(False)
            plain = engines[p].forward(b1025)
            engines[p].set_ln_fold(True)
            folded = engines[p].forward(b1025)
            if p == "fp32":
                assert np.array_equal(folded, plain), p
                continue
            d = np.abs(folded.astype(np.float64) - plain)
            print(f"ln fold, fp16 1025 tokens: max |dlogit| folded vs LayerNorm kernels {float(d.max()):.3g}", flush=True)
            assert not np.array_equal(folded, plain), p
            compare(folded, plain.astype(np.float64), b1025, p)
            for i in (0, 1):
                compare(folded[off1025[i]: off1025[i + 1]], orc.forward([b1025[i]]), [b1025[i]], p)
    finally:
        eng.set_ln_fold(True)
        eng.set_stream_split(8192)


def test_argmax_agreement_1000_requests(base, engines):
    """1,000 requests (500 shaped like cfg2, 500 like cfg5, seeds 10000+i) in
    one batched forward against the oracle's logits in
    tests/golden/argmax_1000.npz (written by make_argmax_fixture.py in this
    directory).

    fp32 validation build, float32 weights: the north-star bars, every argmax
    and max |dp| <= 1e-5.

    fp16 build with certified argmax (dn_set_certify, margin 1e-3: requests
    whose two best logits are closer are recomputed on the fp32 twin): the
    north-star bars, argmax agreement >= 99.9% and max |dp| <= 2e-3, against
    the reference's float32-weight logits, and, loaded with the projection
    weights rounded to bf16 (a BF16 bundle's values), against the oracle run
    on those same weights.

    The raw 16-bit builds, for the record (max |dp| <= 2e-3 and the argmax of
    every decisive request, the oracle's top two probabilities more than
    2 x 2e-3 apart): fp16 against the oracle on the same fp16-rounded weights
    and against the float32-weight logits, 99.7-99.8%; bf16 (its LayerNorms
    folded into the GEMMs, dn_set_ln_fold) against the float32-weight and
    bf16-weight logits, 98.9-99.1% (99.3-99.5% with the LayerNorm kernels).
    Rounding every stored activation to 16 bits moves these random-init
    logits' top-two gaps by ~1.2e-4 (fp16) / ~1e-3 (bf16) RMS, and 19 of the
    1,000 requests have a gap under 1e-3: no 16-bit format reaches 99.9% on
    them unaided, the flips are all such near-ties, and which of them flip
    follows the rounding's particular errors; the RMS error of the top-two
    gap is the steadier measure and is bounded too (bf16: 9.5e-4 folded,
    9.9e-4 with the LayerNorm kernels)."""
    import importlib.util

    from conftest import GOLDEN

    spec = importlib.util.spec_from_file_location("make_argmax_fixture",
                                                  os.path.join(GOLDEN, "make_argmax_fixture.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    cfg = base[0]
    batch = mk.requests(cfg.vocab)
    fx = np.load(os.path.join(GOLDEN, "argmax_1000.npz"))
    assert np.array_equal(np.concatenate([s.ids for s in batch]), fx["ids"])  # same requests as the fixture
    groups = [[(0, len(s.mask_pos))] for s in batch]
    offs = np.concatenate([[0], np.cumsum([len(s.mask_pos) for s in batch])])
    from decide_amd import Engine

    got = {p: engines[p].forward(batch) for p in ("fp32", "bf16", "fp16")}
    w = base[1]
    wb = mk.bf16_projection_weights(w)
    for name, weights in (("fp16+certify", w), ("fp16+certify/bf16w", wb)):
        with Engine(cfg, weights, precision="fp16", certify=1e-3) as ce:
            got[name] = ce.forward(batch)
            print(f"{name}: sequences checked / recomputed {ce.read_certify()}", flush=True)
    for p, key, dp_bar, agree_bar in (("fp32", "logits_f32w", 1e-5, 1.0),
                                      ("fp16+certify", "logits_f32w", 2e-3, 0.999),
                                      ("fp16+certify/bf16w", "logits_bf16w", 2e-3, 0.999),
                                      ("fp16", "logits_f16w", 2e-3, 0.995), ("fp16", "logits_f32w", 2e-3, 0.995),
                                      ("bf16", "logits_f32w", 2e-3, 0.985), ("bf16", "logits_bf16w", 2e-3, 0.985)):
        want = fx[key].astype(np.float64)
        assert got[p].shape == want.shape and np.all(np.isfinite(got[p]))
        pg, pw = _question_probs(got[p], groups), _question_probs(want, groups)
        dp = max(float(np.max(np.abs(a - b))) for a, b in zip(pg, pw))
        flips = [i for i, (a, b) in enumerate(zip(pg, pw)) if np.argmax(a) != np.argmax(b)]
        agree = 1.0 - len(flips) / len(batch)
        top2 = np.array([np.diff(np.sort(b)[-2:])[0] for b in pw])
        decisive = top2 > 2 * dp_bar
        # RMS error of each request's top-two logit gap (the oracle's top two)
        gap_err = []
        for i in range(len(batch)):
            g, r = got[p][offs[i]: offs[i + 1]].astype(np.float64), want[offs[i]: offs[i + 1]]
            t = np.argsort(r)[::-1]
            gap_err.append((g[t[0]] - g[t[1]]) - (r[t[0]] - r[t[1]]))
        rms = float(np.sqrt(np.mean(np.square(gap_err))))
        print(f"1000 requests {p} vs {key}: max|dp| {dp:.3g}, argmax agree {agree:.4f} (flipped {flips}, "
              f"oracle top-2 prob gaps {[float(f'{top2[i]:.2g}') for i in flips]}; {int(decisive.sum())} decisive), "
              f"top-2 logit gap error RMS {rms:.3g}", flush=True)
        assert dp <= dp_bar
        assert agree >= agree_bar
        assert rms <= {"fp32": 1e-5, "bf16": 1.05e-3}.get(p, 2e-4)  # fp16 with or without certification: 2e-4
        assert not any(decisive[i] for i in flips)


def test_stream_split_matches_single_stream(base, engines):
    """dn_set_stream_split: a batch run in two parts on two streams gives the
    single-stream forward's logits bit for bit (each kernel sees the same
    tokens; parts above 1024 tokens run the same GEMM kernels), for the cfg3
    batch, an odd, ragged batch and one whose cut falls after a long
    sequence (2816 tokens, then 20 x 64); through dn_forward and
    dn_forward_device."""
    import torch

    from decide_amd.nn import build_sequence, flatten, row_tokens
    from decide_amd.synth import config_batch, pack_request

    cfg = base[0]
    rng = np.random.default_rng(77)
    ragged = [build_sequence(pack_request(rng, int(p), [int(k)] * int(m), cfg.vocab), 50284, True)
              for p, k, m in zip(rng.integers(40, 900, 9), rng.integers(3, 20, 9), rng.integers(1, 9, 9))]
    lopsided = config_batch("cfg4", vocab=cfg.vocab, nseq=1) + config_batch("cfg5", vocab=cfg.vocab) * 20
    for p in ("bf16", "fp16", "fp32"):
        eng = engines[p]
        for batch in (config_batch("cfg3", vocab=cfg.vocab), ragged, lopsided):
            eng.set_stream_split(0)
            one = eng.forward(batch)
            eng.set_stream_split(1)
            two = eng.forward(batch)
            assert np.array_equal(one, two), (p, len(batch), float(np.max(np.abs(one - two))))
            seq_len, ids, pos, opt, nmask, _ = flatten(batch)
            d = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=ids, pos=pos, opt=opt,
                                                                 rt=row_tokens(batch)).items()}
            out = torch.zeros(len(one), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            eng.forward_device(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(), len(one),
                               d["rt"].data_ptr(), out.data_ptr())
            eng.check_device_errors()
            assert np.array_equal(out.cpu().numpy(), one)
        eng.set_stream_split(8192)


def test_row_tail_matches_full_last_layer(base, engines):
    """dn_set_row_tail: finishing the last layer on the option rows only (their
    attention output and residual rows gathered; Wo, mlp_norm, Wi and MlpWo
    on R rows) gives the logits of the full layer, whose other rows the head
    never reads: the cfg3 batch on one and two streams, the cfg4 batch and a
    ragged batch; through dn_forward and dn_forward_device. The smaller GEMMs
    may sum in another order (fp32: the small-M kernel), so the bar is the
    fp32 rounding bar (|d| <= 1e-5 * (1 + |logit|)) in fp32 and the bf16 bar
    in bf16; the figures are printed."""
    import torch

    from decide_amd.nn import build_sequence, flatten, row_tokens
    from decide_amd.synth import config_batch, pack_request

    cfg = base[0]
    rng = np.random.default_rng(78)
    ragged = [build_sequence(pack_request(rng, int(p), [int(k)] * int(m), cfg.vocab), 50284, True)
              for p, k, m in zip(rng.integers(200, 900, 7), rng.integers(3, 20, 7), rng.integers(1, 9, 7))]
    for p in ("bf16", "fp16", "fp32"):
        eng = engines[p]
        for name, batch, split in (("cfg3", config_batch("cfg3", vocab=cfg.vocab), 1),
                                   ("cfg3", config_batch("cfg3", vocab=cfg.vocab), 0),
                                   ("cfg4", config_batch("cfg4", vocab=cfg.vocab), 8192), ("ragged", ragged, 0)):
            assert sum(len(s.ids) for s in batch) >= 2048
            eng.set_stream_split(split)
            eng.set_row_tail(0)
            full = eng.forward(batch)
            eng.set_row_tail(2048)
            tail = eng.forward(batch)
            d = np.abs(tail.astype(np.float64) - full)
            print(f"row tail {p} {name} split {split}: {len(tail)} rows, bit-identical {np.array_equal(tail, full)}, "
                  f"max |dlogit| {float(d.max()):.3g}", flush=True)
            if p == "fp32":
                assert np.all(d <= 1e-5 * (1 + np.abs(full)))
            else:
                compare(tail, full.astype(np.float64), batch, p)
            seq_len, ids, pos, opt, nmask, _ = flatten(batch)
            dv = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=ids, pos=pos, opt=opt,
                                                                  rt=row_tokens(batch)).items()}
            out = torch.zeros(len(tail), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            eng.forward_device(seq_len, dv["ids"].data_ptr(), dv["pos"].data_ptr(), dv["opt"].data_ptr(), len(tail),
                               dv["rt"].data_ptr(), out.data_ptr())
            eng.check_device_errors()
            assert np.array_equal(out.cpu().numpy(), tail)
        eng.set_stream_split(8192)


def test_row_tail_flags_bad_row_index(base, engines):
    """With the last layer finished on the option rows, dn_forward_device's
    row indices are checked by the row gather: one outside [0, T) is reported
    by dn_check_device_errors as forward.go's mask-position error, and the
    context stays usable."""
    import torch

    from decide_amd import InvalidArgument
    from decide_amd.nn import flatten, row_tokens
    from decide_amd.synth import config_batch

    eng = engines["bf16"]
    batch = config_batch("cfg4", vocab=base[0].vocab, nseq=1)
    want = eng.forward(batch)
    seq_len, ids, pos, opt, nmask, _ = flatten(batch)
    good = row_tokens(batch)
    bad = good.copy()
    bad[3] = len(ids)
    for rt in (bad, good):
        dv = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=ids, pos=pos, opt=opt, rt=rt).items()}
        out = torch.zeros(len(want), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        eng.forward_device(seq_len, dv["ids"].data_ptr(), dv["pos"].data_ptr(), dv["opt"].data_ptr(), len(want),
                           dv["rt"].data_ptr(), out.data_ptr())
        if rt is bad:
            with pytest.raises(InvalidArgument) as ei:
                eng.check_device_errors()
            assert ei.value.message == "nn: mask position out of range"
        else:
            eng.check_device_errors()
            assert np.array_equal(out.cpu().numpy(), want)


def test_row_tail_few_rows_many_sequences(base, engines):
    """dn_forward_device and its no-alloc form accept fewer head rows than
    sequences. With 200 sequences of 12 tokens (2,400 tokens, so the last
    layer runs on the rows) and one or three rows, the option-row attention's
    work list (one item per sequence that holds rows, plus one per 128 rows)
    fits the head scratch whatever the sequence count; each row's logit is
    the full forward's for that token (fp32: |d| <= 1e-5 * (1 + |logit|))."""
    import torch

    from decide_amd.nn import build_sequence, flatten, row_tokens
    from decide_amd.synth import pack_request

    cfg = base[0]
    rng = np.random.default_rng(91)
    batch = [build_sequence(pack_request(rng, 7, [5], cfg.vocab), 50284, True) for _ in range(200)]
    assert sum(len(s.ids) for s in batch) >= 2048
    eng = engines["fp32"]
    eng.set_row_tail(2048)
    full = eng.forward(batch)
    seq_len, ids, pos, opt, nmask, _ = flatten(batch)
    rt_all = row_tokens(batch)
    for pick in ([0], [17, 120, 199]):
        rt = rt_all[pick].astype(np.int32)
        dv = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=ids, pos=pos, opt=opt, rt=rt).items()}
        for fn in (eng.forward_device, eng.forward_device_noalloc):
            out = torch.full((len(rt),), float("nan"), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            fn(seq_len, dv["ids"].data_ptr(), dv["pos"].data_ptr(), dv["opt"].data_ptr(), len(rt),
               dv["rt"].data_ptr(), out.data_ptr())
            eng.synchronize()
            eng.check_device_errors()
            got = out.cpu().numpy().astype(np.float64)
            want = full[pick].astype(np.float64)
            print(f"{fn.__name__} rows {pick}: max |dlogit| {float(np.max(np.abs(got - want))):.3g}", flush=True)
            assert np.all(np.abs(got - want) <= 1e-5 * (1 + np.abs(want)))
    assert np.array_equal(eng.forward(batch), full)


def test_row_tail_gather_fallbacks(base, engines):
    """The row tail's other form (attention over every token, then the
    option rows' attention output gathered), taken for batches of more than
    1,024 sequences and for geometries the MFMA kernels do not tile: logits
    of the full last layer, in both modes (fp32: |d| <= 1e-5 * (1 + |logit|);
    bf16: the bf16 bar)."""
    from decide_amd import Engine, NoGPUError
    from decide_amd.nn import Config, build_sequence
    from decide_amd.synth import config_batch, random_weights

    cfg = base[0]
    many = config_batch("cfg5", vocab=cfg.vocab) * 1100  # 1,100 sequences, 70,400 tokens, 2,200 rows
    small_cfg = Config(hidden=96, intermediate=80, heads=6, layers=3, vocab=300, half_window=8,
                       layer_types=["full_attention", "sliding_attention", "full_attention"])
    rng = np.random.default_rng(11)
    generic = []
    for _ in range(8):  # 8 x ~300 tokens
        ids = [1] + list(rng.integers(3, 299, size=280)) + [2]
        for ln in (4, 5, 6):
            ids += [299] + list(rng.integers(3, 299, size=ln - 1))
        generic.append(build_sequence(np.array(ids + [2], np.int32), 299, independent=True))
    try:
        small = {p: Engine(small_cfg, random_weights(small_cfg, seed=9, std=0.05), precision=p)
                 for p in ("fp32", "bf16")}
    except NoGPUError:
        pytest.skip("no GPU")
    try:
        cases = [("1100 sequences", engines["bf16"], many, "bf16"), ("1100 sequences", engines["fp32"], many, "fp32"),
                 ("generic geometry", small["fp32"], generic, "fp32"),
                 ("generic geometry", small["bf16"], generic, "bf16")]
        for name, eng, batch, p in cases:
            assert sum(len(s.ids) for s in batch) >= 2048
            eng.set_row_tail(0)
            full = eng.forward(batch)
            eng.set_row_tail(2048)
            tail = eng.forward(batch)
            d = np.abs(tail.astype(np.float64) - full)
            print(f"row tail fallback, {name} {p}: {len(tail)} rows, bit-identical {np.array_equal(tail, full)}, "
                  f"max |dlogit| {float(d.max()):.3g}", flush=True)
            if p == "fp32":
                assert np.all(d <= 1e-5 * (1 + np.abs(full)))
            else:
                compare(tail, full.astype(np.float64), batch, p)
    finally:
        for e in small.values():
            e.close()


@pytest.mark.parametrize("layer_types", [["full_attention"], ["full_attention", "sliding_attention"]],
                         ids=["one_layer", "sliding_last"])
def test_row_tail_other_last_layers(layer_types):
    """The option-row last layer when that layer is layer 0 (its QKV input is
    the embedding norm) and when it is a sliding-window layer (the list-mode
    attention with the window test), on a small MFMA geometry (hidden 256, 4
    heads of 64) over 2,600 tokens: the logits of the full last layer up to
    the small-M GEMM kernel's summation order (36 rows; |d| <= 1e-5 * (1 +
    |logit|)), and of the oracle within the bars."""
    from decide_amd import Engine, NoGPUError
    from decide_amd.nn import Config, build_sequence
    from decide_amd.synth import random_weights

    cfg = Config(hidden=256, intermediate=384, heads=4, layers=len(layer_types), vocab=400, half_window=16,
                 layer_types=layer_types)
    w = random_weights(cfg, seed=13, std=0.05)
    rng = np.random.default_rng(14)
    batch = []
    for prem in (900, 700, 500, 300):  # 4 sequences, ~2,600 tokens, 36 option rows
        ids = [1] + list(rng.integers(3, 399, size=prem)) + [2]
        for ln in (5, 9, 17, 3, 12, 7, 20, 4, 6):
            ids += [399] + list(rng.integers(3, 399, size=ln - 1))
        batch.append(build_sequence(np.array(ids + [2], np.int32), 399, independent=True))
    assert sum(len(s.ids) for s in batch) >= 2048
    oracle.set_workers(WORKERS)
    want = oracle.OracleModel(cfg, w).forward(batch)
    for p in ("bf16", "fp32"):
        try:
            eng = Engine(cfg, w, precision=p)
        except NoGPUError:
            pytest.skip("no GPU")
        with eng:
            eng.set_row_tail(0)
            full = eng.forward(batch)
            eng.set_row_tail(2048)
            tail = eng.forward(batch)
        d = np.abs(tail.astype(np.float64) - full)
        print(f"{layer_types} {p}: bit-identical {np.array_equal(tail, full)}, max |dlogit| {float(d.max()):.3g}",
              flush=True)
        assert np.all(d <= 1e-5 * (1 + np.abs(full)))
        if p == "bf16":
            # probabilities only: this random one- or two-layer model's options are near ties
            # (logits within ~0.04), so argmax is not a meaningful bf16 check here
            wb = {n: (a if not n.endswith(("attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight"))
                      else _bf16_round(a)) for n, a in w.items()}
            ref = oracle.OracleModel(cfg, wb).forward(batch)
            dp = max(float(np.max(np.abs(a - b))) for a, b in zip(probs_per_seq(tail, batch), probs_per_seq(ref, batch)))
            print(f"bf16 against the oracle (bf16 weights): max |dp| {dp:.3g}", flush=True)
            assert dp <= 2e-3
        else:
            compare(tail, want, batch, p)


def _bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(np.shape(a))
