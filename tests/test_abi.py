"""CPU checks of the C ABI: the library loads, exports every symbol the header
declares, and its host-side helpers agree with the oracle. No kernel runs."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from conftest import ROOT


def header_symbols():
    text = open(os.path.join(ROOT, "include", "decide_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(dn_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from decide_amd import native

    declared = header_symbols()
    assert len(declared) >= 18
    for name in declared:
        assert hasattr(native.lib, name), name
    assert sorted(native.exported_symbols()) == declared
    assert native.lib.dn_abi_version() == 1


def test_status_strings():
    from decide_amd import native

    assert native.lib.dn_status_string(native.DN_NO_GPU) == b"no GPU"
    assert native.lib.dn_status_string(99) == b"unknown status"


def test_open_without_gpu_is_no_gpu():
    """dn_open maps 'no device' to DN_NO_GPU (the reference's ErrNoGPU path)."""
    from decide_amd import native

    h = ctypes.c_void_p()
    rc = native.lib.dn_open(0, ctypes.byref(h))
    if rc == native.DN_OK:  # running where a GPU exists
        native.lib.dn_close(h)
        pytest.skip("a GPU is present")
    assert rc == native.DN_NO_GPU
    assert b"no GPU" in native.lib.dn_last_error(None)
    assert native.lib.dn_open(0, None) == native.DN_INVALID_ARG


def test_null_context_is_invalid():
    from decide_amd import native

    assert native.lib.dn_forward(None, 0, None, None, None, None, None, None, None, 0) == native.DN_INVALID_ARG
    assert native.lib.dn_set_config(None, 768, 1152, 12, 22, 50368, 1e-5, 64, 1.6e5, 1e4, None, 1) == \
        native.DN_INVALID_ARG


@pytest.mark.parametrize("independent", [False, True])
def test_build_sequence_matches_oracle(independent):
    from decide_amd.nn import build_sequence

    rng = np.random.default_rng(7)
    for trial in range(50):
        n = int(rng.integers(1, 60))
        ids = rng.integers(0, 6, size=n).astype(np.int32)  # mask id 5 appears often
        s = build_sequence(ids, 5, independent)
        p, o, m = oracle.build_sequence(ids, 5, independent)
        assert np.array_equal(s.pos, p) and np.array_equal(s.mask_pos, m)
        assert (s.opt is None) == (o is None)
        if o is not None:
            assert np.array_equal(s.opt, o)


def test_answer_matches_oracle():
    from decide_amd import local

    rng = np.random.default_rng(8)
    for k in (1, 2, 3, 5, 8):
        for t in (0.0, 0.5, 1.0, 2.0):
            logits = rng.standard_normal(k).astype(np.float32)
            if k > 2:
                logits[2] = logits[1]  # a tie
            p, ch, cf = local.answer(logits, t)
            x = logits.astype(np.float64)
            pw = oracle.calibrated(x, t)
            assert np.array_equal(p, pw)
            assert ch == oracle.argmax(x)
            assert cf == oracle.margin_confidence(pw)
    assert local.round_even(0.00015, 4) == oracle.round_even(0.00015, 4)
    assert local.choice_answer(["a", "b"], [0.0, 0.0])["probabilities"] == {"a": 0.5, "b": 0.5}
    assert local.noul_answer([5.0, -5.0])["noul"] == 1.0


def test_config_defaults():
    """LoadConfig defaults (config.go:57-90) on local_test.go's tiny config."""
    from decide_amd.nn import config_from_dict

    c = config_from_dict({"hidden_size": 32, "intermediate_size": 48, "num_attention_heads": 4,
                          "num_hidden_layers": 4, "vocab_size": 300, "norm_eps": 1e-5, "local_attention": 8,
                          "global_attn_every_n_layers": 3, "global_rope_theta": 160000.0,
                          "local_rope_theta": 10000.0})
    assert c.half_window == 4 and c.sliding == [False, True, True, False]
    d = config_from_dict({"hidden_size": 768, "intermediate_size": 1152, "num_attention_heads": 12,
                          "num_hidden_layers": 22, "vocab_size": 50368})
    assert d.eps == 1e-5 and d.half_window == 64 and d.global_theta == 160000 and d.local_theta == 10000
    assert [i for i, s in enumerate(d.sliding) if not s] == [0, 3, 6, 9, 12, 15, 18, 21]
    with pytest.raises(ValueError):
        config_from_dict({"hidden_size": 30, "num_attention_heads": 4, "num_hidden_layers": 1})


def test_synthetic_requests_layout():
    from decide_amd.nn import CLS_ID, MASK_ID, SEP_ID
    from decide_amd.synth import config_batch

    for name, (nseq, n, k) in {"cfg2": (1, 112, 3), "cfg3": (64, 512, 8), "cfg4": (8, 2816, 84),
                               "cfg5": (1, 64, 2)}.items():
        b = config_batch(name)
        assert len(b) == nseq
        for s in b:
            assert len(s.ids) == n and len(s.mask_pos) == k
            assert s.ids[0] == CLS_ID and s.ids[-1] == SEP_ID and s.opt[-1] == -1
            assert int((s.ids == MASK_ID).sum()) == k
            assert not np.any((s.ids >= 50280) & (s.ids <= 50284) & (s.ids != CLS_ID) & (s.ids != SEP_ID)
                              & (s.ids != MASK_ID))
