"""decide.Local on the GPU: a SystemOne call answered with ONE batched
forward (dn_evaluate), against the oracle's restatement of Local.Evaluate,
which runs one Forward per question as the reference does (local.go:126-204).
Also: BF16 bundles (bf16 bits uploaded as stored) and the error paths.

Bars: fp32 mode, rounded probabilities within 1e-4 (one unit of the
4th place, since a 1e-6 difference can cross a rounding boundary), Score
expectation within 0.01, confidence within 0.001, the same choice; bf16
and fp16 modes, probabilities within 2e-3 plus one rounding unit. The fp32
cases pin the batching itself."""
import json
import os

import numpy as np
import pytest

import oracle
import oracle.tokenizer
from test_local import MIN_MASK, byte_encode

pytestmark = pytest.mark.gpu

TINY = {"hidden_size": 256, "intermediate_size": 384, "num_attention_heads": 4, "num_hidden_layers": 4,
        "vocab_size": 300, "norm_eps": 1e-5, "local_attention": 8, "global_attn_every_n_layers": 3,
        "global_rope_theta": 160000.0, "local_rope_theta": 10000.0}
CAL = {"temperature": {"choice": 2.0, "noul": 1.5, "score": 3.0}, "default": 1.0}
STATE = [("ticket", "Payment failed twice"), ("tier", "enterprise")]


def questions():
    from decide_amd.local import Choice, Level, Noul, NoulCriteria, Option, Score, levels

    return [
        ("c", Choice("Which team?", [Option("billing", "Invoices and payments"), Option("tech", "Bugs"),
                                     Option("sales")])),
        ("n", Noul("Is it urgent?")),
        ("n2", Noul("Is it urgent?", NoulCriteria("Urgent", "Routine"))),
        ("s", Score("How severe?", levels("low", "medium", "high"))),
        ("s5", Score("Rate it", [Level("1"), Level("2"), Level("3", ["ok", "fine"]), Level("4"), Level("5")])),
        ("one", Choice("Only one", [Option("only")])),
        ("none", Choice("Nothing", [])),
        ("c2", Choice("Pick a colour for the long-running ticket", [Option(k) for k in "red green blue".split()])),
    ]


@pytest.fixture(scope="module")
def bundles(tmp_path_factory):
    """tinyBundle (local_test.go:20-44) at a geometry the device implements
    (head_dim 64): F32 and BF16 model.safetensors."""
    from decide_amd import bundle, nn
    from decide_amd.synth import random_weights

    cfg = nn.config_from_dict(TINY)
    w = random_weights(cfg, seed=7, std=0.05)
    out = {}
    for dt in ("F32", "BF16"):
        d = tmp_path_factory.mktemp("bundle_" + dt)
        with open(d / "config.json", "w") as fh:
            json.dump(TINY, fh)
        with open(d / "decide.json", "w") as fh:
            json.dump({"name": "decide", "model_id": "decide-test-0", "format": 1, "independent_options": True,
                       "max_tokens": 8192, "calibration": CAL}, fh)
        bundle.write_safetensors(str(d / "model.safetensors"), w, dtype=dt, metadata={"format": "pt"})
        (d / "tokenizer.json").write_bytes(oracle.tokenizer.minimal_json())
        stored, _ = bundle.read_safetensors(str(d / "model.safetensors"))
        wf = {k: bundle.to_float32(*stored[k][::2]).reshape(stored[k][1]) for k in w}
        out[dt] = (str(d), cfg, oracle.OracleModel(cfg, wf))
    return out


def oracle_answers(model, state_text, qs):
    from decide_amd import local as L

    cal = L.Calibration(CAL["temperature"], CAL["default"])
    out = {}
    for qid, q in qs:
        kind, texts, ck = L._options(q)
        name = {L.DN_KIND_CHOICE: "choice", L.DN_KIND_SCORE: "score", L.DN_KIND_NOUL: "noul"}[kind]
        ids = byte_encode(L.pack_text(state_text, q.instructions, texts)) if (name == "noul" or len(texts) > 1) else []
        out[qid] = oracle.evaluate_question(model, name, len(texts), ids, MIN_MASK, True, cal.temperature_for(ck))
    return out


def check_answers(resp, want, qs, prec):
    from decide_amd import local as L

    dp = 1e-4 + 1e-9 if prec == "fp32" else 2e-3 + 1e-4
    worst = 0.0
    for qid, q in qs:
        a, o = resp["answers"][qid], want[qid]
        kind = L._options(q)[0]
        if kind == L.DN_KIND_NOUL:
            assert abs(a["noul"] - o["value"]) <= dp, (qid, a, o)
            continue
        got = list(a["probabilities"].values())
        assert len(got) == len(o["probs"]), qid
        if got:
            worst = max(worst, float(np.max(np.abs(np.array(got) - o["probs"]))))
            assert np.all(np.abs(np.array(got) - o["probs"]) <= dp), (qid, got, o["probs"])
            assert abs(a["confidence"] - o["confidence"]) <= 1e-3 + dp * len(got), (qid, a, o)
        if kind == L.DN_KIND_CHOICE and got:
            assert a["choice"] == [opt.key for opt in q.criteria][o["choice"]], (qid, a, o)
        if kind == L.DN_KIND_SCORE and got:
            assert abs(a["score"] - o["value"]) <= 0.01 + dp * len(got) ** 2, (qid, a, o)
    print(f"{prec}: worst |dp| (rounded) {worst:.3g}", flush=True)


@pytest.mark.parametrize("prec,dt,cert", [("fp32", "F32", 0), ("bf16", "BF16", 0), ("fp32", "BF16", 0),
                                          ("fp16", "F32", 0), ("fp16", "BF16", 0), ("fp16", "BF16", 1e-3)])
def test_system_one_matches_serial_oracle(bundles, prec, dt, cert):
    """The oracle runs the weights the bundle stores (BF16 widened exactly),
    so in bf16 mode only the activation rounding differs. cert: the certified
    argmax's margin (dn_set_certify)."""
    from decide_amd import bundle
    from decide_amd.local import format_state

    d, cfg, om = bundles[dt]
    print(f"case: system_one {prec} {dt} bundle, certify {cert}", flush=True)
    loc = bundle.load_bundle(d, precision=prec, encoder=(byte_encode, MIN_MASK), certify=cert)
    qs = questions()
    resp = loc.system_one(STATE, qs)
    assert resp["model"] == "decide-test-0" and resp["order"] == [q for q, _ in qs]
    check_answers(resp, oracle_answers(om, format_state(STATE), qs), qs, prec)
    c = resp["answers"]["c"]
    assert abs(sum(c["probabilities"].values()) - 1) <= 5e-4 and 0 <= c["confidence"] <= 1
    assert resp["answers"]["one"] == {"choice": "only", "probabilities": {"only": 1.0}, "confidence": 1.0}
    assert resp["answers"]["none"]["probabilities"] == {}
    assert 0 <= resp["answers"]["s"]["score"] <= 2 and len(resp["answers"]["s"]["legend"]) == 3
    # Determinism: the same call again gives the same answers.
    assert loc.system_one(STATE, qs)["answers"] == resp["answers"]
    loc.engine.close()


@pytest.mark.parametrize("prec", ["fp32", "bf16", "fp16"])
def test_many_questions_long_state(bundles, prec):
    """24 questions over a ~1500-token state: one forward of 24 sequences
    (the GEMMs take the large-M path) against 24 serial oracle forwards."""
    from decide_amd import bundle
    from decide_amd.local import Choice, Noul, Option, Score, levels

    d, cfg, om = bundles["BF16" if prec == "bf16" else "F32"]
    rng = np.random.default_rng(3)
    words = ["alpha", "beta", "gamma", "delta", "payment", "failed", "error", "login", "refund", "urgent"]
    state = " ".join(rng.choice(words, size=250))
    qs = []
    for i in range(24):
        if i % 3 == 0:
            qs.append((f"q{i}", Choice(f"choice {i}?", [Option(f"k{j}", " ".join(rng.choice(words, size=3)))
                                                        for j in range(4)])))
        elif i % 3 == 1:
            qs.append((f"q{i}", Noul(f"is {i} true?")))
        else:
            qs.append((f"q{i}", Score(f"rate {i}", levels("a", "b", "c", "d", "e"))))
    print(f"case: 24 questions {prec}", flush=True)
    loc = bundle.load_bundle(d, precision=prec, encoder=(byte_encode, MIN_MASK))
    resp = loc.system_one(state, qs)
    check_answers(resp, oracle_answers(om, state, qs), qs, prec)
    loc.engine.close()


@pytest.mark.parametrize("prec", ["fp32", "bf16", "fp16"])
def test_bf16_upload_equals_widened_f32(bundles, prec):
    """dn_upload_tensor_bf16(bits) gives the same device model as
    dn_upload_tensor(widen(bits)): identical logits, bit for bit."""
    from decide_amd import bundle, nn

    d, cfg, _ = bundles["BF16"]
    stored, _ = bundle.read_safetensors(os.path.join(d, "model.safetensors"))
    a = nn.Engine(cfg, precision=prec)
    b = nn.Engine(cfg, precision=prec)
    for name in nn.tensor_shapes(cfg):
        dt, shape, raw = stored[name]
        a.upload(name, bundle.to_float32(dt, raw))
        b.upload_bf16(name, raw)
    rng = np.random.default_rng(1)
    batch = []
    for n, k in ((40, 2), (300, 4), (129, 3)):
        ids = list(rng.integers(0, 256, size=n))
        for _ in range(k):
            ids += [MIN_MASK] + list(rng.integers(0, 256, size=5))
        batch.append(nn.build_sequence(np.array(ids + [257], np.int32), MIN_MASK, True))
    print(f"case: bf16 upload {prec}", flush=True)
    la, lb = a.forward(batch), b.forward(batch)
    assert np.array_equal(la, lb)
    a.close()
    b.close()


def test_evaluate_errors(bundles):
    """Per-question errors name the first failing question by id; after an
    error the engine still answers (local_test.go:118-140)."""
    from decide_amd import bundle
    from decide_amd.local import Choice, Noul, Option
    from decide_amd.native import InvalidArgument

    d, _, _ = bundles["F32"]
    loc = bundle.load_bundle(d, precision="bf16", encoder=(byte_encode, MIN_MASK))
    with pytest.raises(InvalidArgument, match="question 'q': input contains the reserved \\[MASK\\] token"):
        # 'one' skips the model, so 'q' is the first question whose input is checked.
        loc.system_one("text with [MASK] injected", [("one", Choice("i", [Option("only")])),
                                                     ("q", Choice("i", [Option("a"), Option("b")])),
                                                     ("n", Noul("fine"))])
    with pytest.raises(InvalidArgument, match="duplicate choice"):
        loc.system_one("s", [("q", Choice("i", [Option("a"), Option("a")]))])
    with pytest.raises(InvalidArgument, match="duplicate question id"):
        loc.system_one("s", [("q", Noul("i")), ("q", Noul("j"))])
    with pytest.raises(InvalidArgument, match="question 'long': input is \\d+ tokens; the limit is 8192"):
        loc.system_one("x" * 8990, [("long", Noul("i"))])
    r = loc.system_one("s", [("q", Choice("i", [Option("only")]))])
    assert r["answers"]["q"] == {"choice": "only", "probabilities": {"only": 1.0}, "confidence": 1.0}
    r = loc.system_one("s", [("q", Noul("i"))])
    assert 0 <= r["answers"]["q"]["noul"] <= 1
    loc.engine.close()


def test_system_one_with_bundle_tokenizer(bundles):
    """load_bundle without an encoder tokenizes with the library's tokenizer
    (the bundle's tokenizer.json, here tokenizer.MinimalJSON): the same
    answers as with the test's byte-level encoder."""
    from decide_amd import bundle

    d, _, _ = bundles["F32"]
    qs = questions()
    a = bundle.load_bundle(d, precision="fp32")
    b = bundle.load_bundle(d, precision="fp32", encoder=(byte_encode, MIN_MASK))
    assert a.mask_id == MIN_MASK
    assert a.system_one(STATE, qs)["answers"] == b.system_one(STATE, qs)["answers"]
    a.engine.close()
    b.engine.close()
