"""Certified argmax (dn_set_certify) on the GPU, through the C ABI.

A 16-bit forward moves each logit by its rounding error; with certification
on, a sequence whose two largest logits are less than the margin apart is
recomputed on the context's fp32 twin. Checked here: the sequences left
alone keep the 16-bit logits bit for bit, the recomputed ones carry the fp32
path's logits (within fp32 rounding of an fp32 engine's), the counters match
the near-ties, dn_forward_device gives dn_forward's certified logits bit for
bit, a margin covering every sequence reproduces the fp32 mode, and the
set-up errors. The agreement rates over 1,000 requests are
test_gpu_forward.test_argmax_agreement_1000_requests'."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MARGIN = 1e-3  # fp16: ~8x the measured RMS error of a logit difference (1.2e-4)


def top2_gaps(logits, batch):
    out, off = [], 0
    for s in batch:
        k = len(s.mask_pos)
        z = np.sort(np.asarray(logits[off: off + k], np.float64))
        out.append(z[-1] - z[-2] if k >= 2 else np.inf)
        off += k
    return np.array(out)


def rows_of(batch):
    out, off = [], 0
    for s in batch:
        k = len(s.mask_pos)
        out.append(slice(off, off + k))
        off += k
    return out


@pytest.fixture(scope="module")
def setup():
    from decide_amd import Engine, NoGPUError, modernbert_base
    from decide_amd.synth import random_weights

    cfg = modernbert_base()
    w = random_weights(cfg, seed=0)
    try:
        engs = {"raw": Engine(cfg, w, precision="fp16"), "cert": Engine(cfg, w, precision="fp16", certify=MARGIN),
                "fp32": Engine(cfg, w, precision="fp32")}
    except NoGPUError:
        pytest.skip("no GPU")
    yield cfg, w, engs
    for e in engs.values():
        e.close()


def _requests(cfg, n, seed):
    from decide_amd.nn import MASK_ID, build_sequence
    from decide_amd.synth import pack_request

    rng = np.random.default_rng(seed)
    return [build_sequence(pack_request(rng, int(rng.integers(20, 90)), [int(rng.integers(3, 20))] * int(k),
                                        cfg.vocab), MASK_ID, True)
            for k in rng.integers(2, 6, size=n)]


def test_certify_replaces_only_near_ties(setup):
    cfg, _, e = setup
    batch = _requests(cfg, 300, 41)
    raw = e["raw"].forward(batch)
    e["cert"].read_certify()
    cert = e["cert"].forward(batch)
    checked, recomputed = e["cert"].read_certify()
    exact = e["fp32"].forward(batch)
    near = top2_gaps(raw, batch) < MARGIN
    print(f"case: certify 300 requests: {int(near.sum())} near-ties, counters {checked} / {recomputed}", flush=True)
    assert checked == len(batch) and recomputed == int(near.sum()) and recomputed > 0
    for i, sl in enumerate(rows_of(batch)):
        if near[i]:
            assert np.all(np.abs(cert[sl].astype(np.float64) - exact[sl]) <= 1e-5 * (1 + np.abs(exact[sl]))), i
            assert np.argmax(cert[sl]) == np.argmax(exact[sl])
        else:
            assert np.array_equal(cert[sl], raw[sl]), i


def test_certify_device_entry_matches_host_entry(setup):
    """dn_forward_device with certification gives dn_forward's certified
    logits bit for bit (the same 16-bit forward, the same sequences recomputed
    by the same fp32 twin): the cfg3 batch (64 x 512, the bench workload) and
    a ragged batch of plain and independent sequences."""
    import torch

    from decide_amd.nn import flatten, row_tokens
    from decide_amd.synth import config_batch

    cfg, _, e = setup
    for name, batch in (("cfg3", config_batch("cfg3", vocab=cfg.vocab)), ("ragged", _requests(cfg, 40, 43))):
        host = e["cert"].forward(batch)
        _, n_host = e["cert"].read_certify()
        seq_len, ids, pos, opt, nmask, _ = flatten(batch)
        d = {k: torch.from_numpy(v).cuda() for k, v in dict(ids=ids, pos=pos, opt=opt, rt=row_tokens(batch)).items()}
        out = torch.full((len(host),), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        e["cert"].forward_device(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(), len(host),
                                 d["rt"].data_ptr(), out.data_ptr())
        e["cert"].synchronize()
        e["cert"].check_device_errors()
        _, n_dev = e["cert"].read_certify()
        print(f"case: certify device entry {name}: recomputed {n_host} (host) / {n_dev} (device)", flush=True)
        assert n_host == n_dev
        assert np.array_equal(out.cpu().numpy(), host)


def test_certify_everything_is_the_fp32_path(setup):
    """A margin larger than every gap sends every sequence to the twin: the
    fp32 mode's logits within fp32 rounding."""
    from decide_amd import Engine

    cfg, w, e = setup
    batch = _requests(cfg, 12, 47)
    with Engine(cfg, w, precision="fp16", certify=1e6) as all_exact:
        got = all_exact.forward(batch)
        assert all_exact.read_certify() == (12, 12)
    want = e["fp32"].forward(batch)
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * (1 + np.abs(want)))


def test_certify_setup_errors(setup):
    from decide_amd import Engine, InvalidArgument, Unsupported
    from decide_amd.train import TrainEngine

    cfg, w, e = setup
    with pytest.raises(InvalidArgument, match="precede the weight uploads"):
        e["raw"].set_certify(MARGIN)
    with pytest.raises(InvalidArgument, match="already the exact path"):
        e["fp32"].set_certify(MARGIN)
    with Engine(cfg, None, precision="fp16") as x:
        with pytest.raises(InvalidArgument, match="margin"):
            x.set_certify(-1.0)
        x.set_certify(MARGIN)
        x.set_certify(0.0)  # off again
    with TrainEngine(cfg, None, precision="bf16") as t:
        with pytest.raises(Unsupported, match="training"):
            t.set_certify(MARGIN)
