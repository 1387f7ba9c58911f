"""CPU checks of the host side around the forward: PackText, formatState,
calibration temperatures, safetensors IO (F32 and BF16) and the oracle's
restatement of Local.Evaluate, pinned by the reference's own test cases.
No kernel runs."""
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN

# tokenizer.MinimalJSON (internal/tokenizer/tokenizer.go:363-395): byte-level
# vocabulary 0-255, no merges, specials [CLS] 256, [SEP] 257, [MASK] 258
# (lstrip), [PAD] 259, [UNK] 260.
MIN_SPECIAL = {"[CLS]": (256, False), "[SEP]": (257, False), "[MASK]": (258, True), "[PAD]": (259, False),
               "[UNK]": (260, False)}
MIN_MASK = 258


def byte_encode(text: str):
    """Encode(text, true) with the MinimalJSON tokenizer (tokenizer.go:133-225):
    leftmost-longest special-token split on the raw text (lstrip trims the
    whitespace before [MASK]), NFC, then one id per UTF-8 byte (no merges)."""
    import unicodedata

    ids = [256]
    rest = text
    while rest:
        best = None
        for tok, (tid, lstrip) in MIN_SPECIAL.items():
            i = rest.find(tok)
            if i >= 0 and (best is None or i < best[0] or (i == best[0] and len(tok) > len(best[1]))):
                best = (i, tok, tid, lstrip)
        if best is None:
            ids += list(unicodedata.normalize("NFC", rest).encode())
            break
        i, tok, tid, lstrip = best
        before = rest[:i].rstrip() if lstrip else rest[:i]
        if before:
            ids += list(unicodedata.normalize("NFC", before).encode())
        ids.append(tid)
        rest = rest[i + len(tok):]
    ids.append(257)
    return ids


def test_pack_text_layout():
    """TestPackTextLayout (internal/train/train_test.go:52-62)."""
    from decide_amd.local import pack_text

    assert pack_text("the state", "Which?", [" a ", "b"]) == "Which? the state [SEP] [MASK] a [MASK] b"
    assert pack_text("only state", "", ["x", "y"]) == "only state [SEP] [MASK] x [MASK] y"


def test_format_state():
    """TestFormatState / TestParseRequest (types_test.go:114, :165-192), the cases
    whose Go value has a Python counterpart."""
    from decide_amd.local import format_state

    assert format_state("plain") == "plain"
    assert format_state([("k", "v"), ("n", 3), ("f", 2.50), ("t", True), ("z", None)]) == \
        "k: v\nn: 3\nf: 2.5\nt: True\nz: None"
    assert format_state([("list", ["a", 1, False]), ("o", {"x": "it's"})]) == "list: ['a', 1, False]\no: {'x': \"it's\"}"
    assert format_state({"b": 1, "a": "x"}) == "b: 1\na: x"  # a decoded JSON object keeps its order
    assert format_state(42) == "42"
    assert format_state(["a", "b"]) == "['a', 'b']"
    assert format_state(None) == "None"


def test_calibration_temperature_for():
    """Calibration.TemperatureFor (internal/bundle/bundle.go:39-50)."""
    from decide_amd.local import Calibration

    c = Calibration({"choice": 2.0, "noul": 0.0}, default=1.5)
    assert c.temperature_for("choice") == 2.0
    assert c.temperature_for("noul") == 1.5  # non-positive fitted value falls back to the default
    assert c.temperature_for("score") == 1.5
    assert Calibration().temperature_for("score") == 1.0


def test_byte_encoder_layout():
    """The MinimalJSON encoding of a packed question: [MASK] strips the space before it."""
    from decide_amd.local import pack_text

    ids = byte_encode(pack_text("st", "q", ["a", "bc"]))
    assert ids == [256] + list(b"q st ") + [257, 258] + list(b" a") + [258] + list(b" bc") + [257]


def test_question_option_texts():
    """Option texts and checks of evalChoice / evalScore / evalNoul (local.go:264-356)."""
    from decide_amd import local as L

    k, texts, cal = L._options(L.Choice("i", [L.Option("a", " Desc "), L.Option(" b ")]))
    assert (k, texts, cal) == (L.DN_KIND_CHOICE, ["Desc", "b"], "choice")
    with pytest.raises(ValueError, match="duplicate choice"):
        L._options(L.Choice("i", [L.Option("a"), L.Option("a")]))
    k, texts, _ = L._options(L.Score("i", [L.Level("low"), L.Level("hi", ["x", "y"])]))
    assert texts == ["low", "hi Examples: x, y"]
    assert L._options(L.Noul("i"))[1] == [L.DEFAULT_YES, L.DEFAULT_NO]
    assert L._options(L.Noul("i", L.NoulCriteria(" Urgent ", "")))[1] == ["Urgent", L.DEFAULT_NO]


# ------------------------------------------------------------------ safetensors
def test_safetensors_roundtrip_f32_bf16(tmp_path):
    """Our writer/reader against the safetensors package (independent
    implementation) and torch's bfloat16 rounding."""
    import torch
    from safetensors.torch import load_file

    from decide_amd import bundle

    rng = np.random.default_rng(0)
    t = {"b.w": rng.standard_normal((3, 5)).astype(np.float32), "a": rng.standard_normal(7).astype(np.float32)}
    t["a"][:3] = [0.0, -0.0, 3.0e38]
    for dt in ("F32", "BF16"):
        path = str(tmp_path / f"m_{dt}.safetensors")
        bundle.write_safetensors(path, t, dtype=dt, metadata={"format": "pt"})
        got, meta = bundle.read_safetensors(path)
        assert meta == {"format": "pt"}
        lib = load_file(path)
        for name, a in t.items():
            d, shape, raw = got[name]
            assert d == dt and shape == a.shape
            want = torch.from_numpy(a).to(torch.bfloat16) if dt == "BF16" else torch.from_numpy(a)
            assert torch.equal(lib[name], want)
            if dt == "BF16":
                assert np.array_equal(raw, want.view(torch.int16).numpy().view(np.uint16).reshape(-1))
                assert np.array_equal(bundle.to_float32(d, raw), want.float().numpy().reshape(-1))
            else:
                assert np.array_equal(raw, a.reshape(-1))
        # header padded to 8 bytes, names sorted
        with open(path, "rb") as fh:
            n = int.from_bytes(fh.read(8), "little")
            assert (8 + n) % 8 == 0


def test_reads_reference_fixture():
    """The reference's tiny_ref.safetensors reads the same through our reader
    and the safetensors package."""
    from safetensors.numpy import load_file

    from decide_amd import bundle

    path = os.path.join(GOLDEN, "tiny_ref.safetensors")
    got, _ = bundle.read_safetensors(path)
    lib = load_file(path)
    assert set(got) == set(lib)
    for name, (dt, shape, raw) in got.items():
        assert np.array_equal(bundle.to_float32(dt, raw).reshape(shape), lib[name].astype(np.float32))


# ------------------------------------------------------- oracle Local.Evaluate
@pytest.fixture(scope="module")
def tiny_local():
    """tinyBundle's model (local_test.go:15-44): tinyConfig geometry,
    random weights, independent options, MinimalJSON tokenizer."""
    from decide_amd.nn import config_from_dict
    from decide_amd.synth import random_weights

    cfg = config_from_dict({"hidden_size": 32, "intermediate_size": 48, "num_attention_heads": 4,
                            "num_hidden_layers": 4, "vocab_size": 300, "norm_eps": 1e-5, "local_attention": 8,
                            "global_attn_every_n_layers": 3, "global_rope_theta": 160000.0,
                            "local_rope_theta": 10000.0})
    w = random_weights(cfg, seed=7, std=0.3)
    return oracle.OracleModel(cfg, w)


def ask(model, kind, state, instr, options, temp=1.0):
    from decide_amd.local import pack_text

    return oracle.evaluate_question(model, kind, len(options), byte_encode(pack_text(state, instr, options)),
                                    MIN_MASK, True, temp)


def test_oracle_local_end_to_end_properties(tiny_local):
    """TestLocalEndToEnd's checks (local_test.go:46-91) on the oracle."""
    c = ask(tiny_local, "choice", "ticket: Payment failed twice", "Which team?",
            ["Invoices and payments", "Bugs", "sales"], 2.0)
    assert abs(sum(c["probs"]) - 1) <= 5e-4 and 0 <= c["confidence"] <= 1
    assert c["probs"][c["choice"]] >= 1 / 3 - 1e-3
    n = ask(tiny_local, "noul", "ticket: Payment failed twice", "Is it urgent?",
            ["Yes, condition holds true.", "No, condition is false."], 1.5)
    assert 0 <= n["value"] <= 1
    s = ask(tiny_local, "score", "ticket: Payment failed twice", "How severe?", ["low", "medium", "high"], 3.0)
    assert 0 <= s["value"] <= 2
    again = ask(tiny_local, "choice", "ticket: Payment failed twice", "Which team?",
                ["Invoices and payments", "Bugs", "sales"], 2.0)
    assert again == c


def test_oracle_local_order_invariant(tiny_local):
    """TestLocalOrderInvariant (local_test.go:93-116): permuting the options
    permutes the probabilities (within 2e-4) and keeps the winner."""
    opts = ["first option text", "second", "the third one", "4th"]
    perm = [2, 0, 3, 1]
    x = ask(tiny_local, "choice", "some state text", "pick", opts)
    y = ask(tiny_local, "choice", "some state text", "pick", [opts[i] for i in perm])
    assert perm[y["choice"]] == x["choice"]
    for j, i in enumerate(perm):
        assert abs(x["probs"][i] - y["probs"][j]) <= 2e-4


def test_oracle_local_errors(tiny_local):
    """TestLocalErrors (local_test.go:118-140) and the single-option shortcut."""
    with pytest.raises(ValueError, match="reserved"):
        ask(tiny_local, "choice", "text with [MASK] injected", "i", ["a", "b"])
    one = oracle.evaluate_question(tiny_local, "choice", 1, [], MIN_MASK, True, 1.0)
    assert one == {"probs": [1.0], "choice": 0, "confidence": 1.0, "value": 0.0}
    s1 = oracle.evaluate_question(tiny_local, "score", 1, [], MIN_MASK, True, 1.0)
    assert s1["probs"] == [1.0] and s1["value"] == 0.0 and s1["confidence"] == 1.0
    with pytest.raises(ValueError, match="limit is 8192"):
        oracle.evaluate_question(tiny_local, "noul", 2, [1] * 8193, MIN_MASK, True, 1.0)
