"""dn_forward_device_noalloc through the C ABI: the same logits as
dn_forward_device, bit for bit, on two calls in a row (the second smaller),
with an ordinary forward in between, and DN_INVALID_ARG past the scratch
array's maximum."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _stage(batch, dev):
    import torch

    from decide_amd.nn import flatten, row_tokens

    seq_len, ids, pos, opt, nmask, _ = flatten(batch)
    d = {k: torch.from_numpy(v).to(dev) for k, v in (("ids", ids), ("pos", pos), ("opt", opt),
                                                       ("rt", row_tokens(batch)))}
    R = int(nmask.sum())
    return seq_len, d, R


def _run(eng, batch, noalloc):
    import torch

    seq_len, d, R = _stage(batch, "cuda")
    out = torch.full((R,), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    fn = eng.forward_device_noalloc if noalloc else eng.forward_device
    fn(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(), R, d["rt"].data_ptr(), out.data_ptr())
    eng.synchronize()
    eng.check_device_errors()
    return out.cpu().numpy()


@pytest.mark.parametrize("precision", ["bf16", "fp16", "fp32"])
def test_noalloc_matches_forward_device(precision):
    from decide_amd import Engine, NoGPUError, modernbert_base
    from decide_amd.synth import config_batch, random_weights

    cfg = modernbert_base()
    try:
        eng = Engine(cfg, random_weights(cfg, seed=3), precision=precision)
    except NoGPUError:
        pytest.skip("no GPU")
    with eng:
        big = config_batch("cfg3", vocab=cfg.vocab, nseq=4, seed=5)  # 4 x 512 tokens, 32 rows
        small = config_batch("cfg5", vocab=cfg.vocab, seed=6)        # 64 tokens, 2 rows
        want_big, want_small = _run(eng, big, False), _run(eng, small, False)
        got_big = _run(eng, big, True)
        mid = _run(eng, small, False)  # an ordinary forward between the two calls
        got_small = _run(eng, small, True)
        assert np.all(np.isfinite(got_big)) and np.all(np.isfinite(got_small))
        assert np.array_equal(got_big, want_big), np.max(np.abs(got_big - want_big))
        assert np.array_equal(got_small, want_small), np.max(np.abs(got_small - want_small))
        assert np.array_equal(mid, want_small)
        # and the ordinary path is undisturbed afterwards
        assert np.array_equal(_run(eng, big, False), want_big)


def test_noalloc_rejects_batches_past_the_scratch_size():
    from decide_amd import Engine, InvalidArgument, NoGPUError, modernbert_base
    from decide_amd.synth import config_batch, random_weights

    cfg = modernbert_base()
    try:
        eng = Engine(cfg, random_weights(cfg, seed=3), precision="bf16")
    except NoGPUError:
        pytest.skip("no GPU")
    with eng:
        huge = config_batch("cfg3", vocab=cfg.vocab, nseq=12, seed=7)  # 6144 tokens > ~5,100
        with pytest.raises(InvalidArgument, match="bytes of scratch; the maximum is 67108864"):
            _run(eng, huge, True)
        # a call that fits still works after the refusal
        ok = config_batch("cfg5", vocab=cfg.vocab, seed=8)
        assert np.array_equal(_run(eng, ok, True), _run(eng, ok, False))


def test_noalloc_first_call_allocates_nothing():
    """A context whose first forward is the no-alloc one: the device's free
    memory is the same before and after the call (a stray context-buffer
    allocation on that path would take it down by the activations' size)."""
    import torch

    from decide_amd import Engine, NoGPUError, modernbert_base
    from decide_amd.synth import config_batch, random_weights

    cfg = modernbert_base()
    w = random_weights(cfg, seed=3)
    batch = config_batch("cfg3", vocab=cfg.vocab, nseq=4, seed=5)
    try:
        warm = Engine(cfg, w, precision="bf16")
    except NoGPUError:
        pytest.skip("no GPU")
    with warm:  # loads the kernels' code objects, which takes device memory once per process
        want = _run(warm, batch, False)
    with Engine(cfg, w, precision="bf16") as eng:
        seq_len, d, R = _stage(batch, "cuda")
        out = torch.full((R,), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        eng.forward_device_noalloc(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(), R,
                                   d["rt"].data_ptr(), out.data_ptr())
        eng.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        eng.check_device_errors()
        assert free1 == free0, (free0, free1)
        assert np.array_equal(out.cpu().numpy(), want)


def test_noalloc_refuses_stream_capture():
    """The no-alloc entry synchronises its stream, so under capture it must
    refuse (DN_UNSUPPORTED) without enqueuing anything; the capture itself
    stays valid and the context works afterwards."""
    import torch

    from decide_amd import Engine, NoGPUError, Unsupported, modernbert_base
    from decide_amd.synth import config_batch, random_weights

    cfg = modernbert_base()
    try:
        eng = Engine(cfg, random_weights(cfg, seed=3), precision="bf16")
    except NoGPUError:
        pytest.skip("no GPU")
    with eng:
        batch = config_batch("cfg5", vocab=cfg.vocab, seed=8)
        want = _run(eng, batch, False)
        seq_len, d, R = _stage(batch, "cuda")
        out = torch.zeros((R,), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        eng.set_stream(s.cuda_stream)
        try:
            with torch.cuda.graph(g, stream=s):
                out.fill_(1.0)
                with pytest.raises(Unsupported, match="stream capture"):
                    eng.forward_device_noalloc(seq_len, d["ids"].data_ptr(), d["pos"].data_ptr(), d["opt"].data_ptr(),
                                               R, d["rt"].data_ptr(), out.data_ptr())
        finally:
            eng.set_stream(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.all(out.cpu().numpy() == 1.0)
        assert np.array_equal(_run(eng, batch, True), want)
