import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libdecide_hip.so)")


@pytest.fixture(scope="session")
def tiny_ref():
    """The reference's PyTorch fixture (internal/nn/testdata/tiny_ref.safetensors,
    written by gen_ref.py): weights under w.<name>, goldens logits/loss/hidden.*/l1.*."""
    from safetensors import safe_open
    from safetensors.numpy import load_file

    path = os.path.join(GOLDEN, "tiny_ref.safetensors")
    tensors = load_file(path)
    with safe_open(path, framework="numpy") as f:
        meta = json.loads(f.metadata()["meta"])
    return tensors, meta


def tiny_config(meta):
    """loadRef's config (internal/nn/nn_test.go:38-43)."""
    from decide_amd.nn import Config

    c = meta["config"]
    return Config(hidden=c["hidden"], intermediate=c["intermediate"], heads=c["heads"], layers=c["layers"],
                  vocab=c["vocab"], eps=1e-5, half_window=c["half_window"],
                  global_theta=c["global_theta"], local_theta=c["local_theta"],
                  layer_types=["full_attention", "sliding_attention", "sliding_attention", "full_attention"])


def tiny_weights(tensors, cfg):
    from decide_amd.nn import tensor_shapes

    return {name: tensors["w." + name].reshape(shape) for name, shape in tensor_shapes(cfg).items()}


def rel_err(got, want):
    """relErr of nn_test.go:95-103: ||got-want|| / (||want|| + 1e-4)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.sqrt(((got - want) ** 2).sum()) / (np.sqrt((want ** 2).sum()) + 1e-4))
