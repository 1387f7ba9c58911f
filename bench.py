"""Benchmark: ModernBERT-base encoder forward on one MI355X.

One step = one dn_forward_device over one batch of the workload (default
cfg3: 64 requests x 512 tokens, 384-token premise + 8 options x 16, the
premise/option block mask, all 22 layers, scorer head), with weights and
token arrays already resident in HBM. Prints one JSON line (see the keys
below). Synthetic data: weights N(0, 0.02) with InitRandom semantics and
seeded token ids; see decide_amd/synth.py.

  python bench.py [--steps K] [--warmup W] [--config cfg3] [--precision bf16]
  python bench.py --systemone [--steps K]   one SystemOne call, batched vs serial
  python bench.py --train [--steps K]       one training step (forward, backward, AdamW)
  python bench.py --tokenizer               host tokenizer throughput (CPU only)
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import re
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "encoder tokens/sec + GEMM TFLOP/s (% bf16 MFMA peak), ModernBERT-base, 1 MI355X"
PEAK = {"bf16": 2.5e15, "fp16": 2.5e15, "fp32": 157.3e12}  # dense MFMA peaks, FLOP/s
H, I = 768, 1152
PROJ_FLOP_PER_TOKEN_LAYER = 2 * H * (3 * H + H + 2 * I + I)  # 10,027,008
WORKLOADS = {
    "cfg2": "cfg2: 1 Choice request x 112 tokens (64-token premise + 3 options x 16)",
    "cfg3": "cfg3: batch 64 x seq 512 (384-token premise + 8 options x 16), block-masked, 22 layers",
    "cfg4": "cfg4: batch 8 x seq 2816 (2048-token premise + 24 question segments, 84 options)",
    "cfg5": "cfg5: batch 1 x seq 64 (40-token premise + 2 options x 12)",
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads() -> int:
    """Host threads of this process's CPU share (the GPU box gives each GPU 16)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_cpu_info() -> dict:
    """nproc, sockets and model of the host CPU (from /proc/cpuinfo)."""
    model, sockets = "unknown", set()
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model == "unknown":
                    model = v
                elif k == "physical id":
                    sockets.add(v)
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {"model": model, "nproc": os.cpu_count(), "sockets": max(1, len(sockets)), "affinity": affinity,
            "threads_used": cpu_threads()}


def cpu_baseline(cfg, weights, name: str, budget_s: float = 12.0, threads: int = None):
    """The oracle (C++ restatement of the reference's Go AVX2 forward) on a
    bounded sample of the same workload: whole sequences of the workload until
    about budget_s seconds of CPU work."""
    import oracle
    from decide_amd.synth import config_batch

    threads = threads or cpu_threads()
    oracle.set_workers(threads)
    model = oracle.OracleModel(cfg, weights)
    full = config_batch(name, vocab=cfg.vocab)
    toks, secs, nseq = 0, 0.0, 0
    while secs < budget_s and nseq < len(full) * 4:
        s = full[nseq % len(full)]
        t0 = time.perf_counter()
        model.forward([s])
        secs += time.perf_counter() - t0
        toks += len(s.ids)
        nseq += 1
    return {"value": round(toks / secs, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{nseq} sequence(s) of {name} ({toks} tokens) one forward per sequence, "
                      f"{secs:.1f} s; C++ restatement of the reference Go AVX2 path (oracle/)"}


def cpu_gemm_cfg1(threads: int, budget_s: float = 3.0) -> dict:
    """cfg1 on the oracle's Go-order sgemm (blas.Sgemm's blocking and job
    queue): GFLOP/s of X[512x768] . W^T, W[2304x768] over about budget_s."""
    import oracle

    rng = np.random.default_rng(0)
    M, N, K = 512, 2304, 768
    X = rng.standard_normal(M * K, dtype=np.float32)
    W = (rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    C = np.zeros(M * N, np.float32)
    secs, n = 0.0, 0
    while secs < budget_s:
        t0 = time.perf_counter()
        oracle.sgemm(False, True, M, N, K, X, K, W, K, C, N, False, workers=threads)
        secs += time.perf_counter() - t0
        n += 1
    return {"gflops": round(2.0 * M * N * K * n / secs / 1e9, 2), "threads": threads, "calls": n}


LIBGEMM_METRIC = ("projection GEMMs alone, back to back: this library's kernels vs hipBLASLt (torch.mm), "
                  "bf16, ModernBERT-base shapes, 1 MI355X")


def library_gemm(args) -> int:
    """Times the forward's four projection shapes in isolation at cfg3's and
    cfg4's token counts: QKV and Wi through dn_gemm_device_store (the plain
    product rounded to bf16: Wi without its GeGLU), Wo and MlpWo through
    dn_gemm_device (fp32 output added to C: the residual read-modify-write),
    against torch.mm (hipBLASLt, bf16 output, no residual) with the activation
    row stride the forward uses (K) and with K + 64. Repetitions alternate the
    three. Back-to-back launches of one kernel run at a lower shader clock than
    the same launch inside a forward, so these figures are not the forward's
    per-launch times. Prints one JSON line."""
    import torch

    from decide_amd import Engine, modernbert_base

    torch.cuda.init()
    eng = Engine(modernbert_base(), None, precision="bf16")  # no weights: the GEMM entry points only
    eng.set_stream(torch.cuda.current_stream().cuda_stream)

    def timed(f, it=20):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(it):
            f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / it * 1e3

    rows = []
    for T, wl in ((32768, "cfg3"), (22528, "cfg4")):
        for name, N, K in (("qkv", 3 * H, H), ("wi", 2 * I, H), ("wo", H, H), ("mlpwo", H, I)):
            g = torch.Generator(device="cuda").manual_seed(T + N + K)
            A = torch.randn(T, K + 64, device="cuda", generator=g).to(torch.bfloat16)
            Bw = (torch.randn(N, K + 64, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
            Ac, Bc = A[:, :K].contiguous(), Bw[:, :K].contiguous()
            Ap, Bp = A[:, :K], Bw[:, :K]  # row stride K + 64
            if name in ("qkv", "wi"):
                C = torch.empty(T, N, device="cuda", dtype=torch.bfloat16)
                ours = lambda: eng.gemm_device_store("bf16", T, N, K, Ac.data_ptr(), Bc.data_ptr(), C.data_ptr())  # noqa: E731
            else:
                C = torch.zeros(T, N, device="cuda", dtype=torch.float32)
                ours = lambda: eng.gemm_device("bf16", T, N, K, Ac.data_ptr(), Bc.data_ptr(), C.data_ptr(), True)  # noqa: E731
            lib = lambda: torch.mm(Ac, Bc.t())  # noqa: E731
            libp = lambda: torch.mm(Ap, Bp.t())  # noqa: E731
            t = {"ours": [], "lib": [], "libp": []}
            for _ in range(3):
                t["ours"].append(timed(ours))
                t["lib"].append(timed(lib))
                t["libp"].append(timed(libp))
            eng.check_device_errors()
            flop = 2.0 * T * N * K
            med = {k: float(np.median(v)) for k, v in t.items()}
            rows.append({"workload": wl, "gemm": name, "M": T, "N": N, "K": K,
                         "ours_us": round(med["ours"], 1), "ours_tflops": round(flop / med["ours"] / 1e6, 1),
                         "hipblaslt_us": round(med["lib"], 1), "hipblaslt_tflops": round(flop / med["lib"] / 1e6, 1),
                         "hipblaslt_lda_k_plus_64_us": round(med["libp"], 1)})
            log(f"{wl} {name}: ours {med['ours']:.1f} us, hipBLASLt {med['lib']:.1f} us (lda K+64: {med['libp']:.1f})")
            del A, Bw, Ac, Bc, C
    print(json.dumps({"metric": LIBGEMM_METRIC, "unit": "us", "higher_is_better": False, "n_gpus": 1,
                      "data": "synthetic: A N(0,1), B N(0,0.02), bf16", "results": rows}))
    eng.close()
    return 0


SYSTEMONE_METRIC = ("SystemOne call: 24 questions (cfg4 mix) over a 2048-token state, answered with one "
                    "batched forward vs one forward per question, ModernBERT-base, 1 MI355X")


def systemone(args) -> int:
    """Times Local.Evaluate's work for one SystemOne call through the C ABI
    (host ids in, answers out, validation and post-processing included):
    dn_evaluate over all 24 questions (one forward) against 24 dn_evaluate
    calls of one question each (one forward per question, as local.go:126-150
    runs them). Prints one JSON line."""
    import ctypes

    from decide_amd import Engine, modernbert_base
    from decide_amd.native import check, lib
    from decide_amd.nn import MASK_ID
    from decide_amd.synth import random_weights, systemone_call

    cfg = modernbert_base()
    weights = random_weights(cfg, seed=0)
    kinds, nopt, qids = systemone_call(cfg.vocab)
    nq = len(kinds)
    eng = Engine(cfg, weights, precision=args.precision)
    h = eng.handle
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731

    def call(sel):
        k = np.array([kinds[i] for i in sel], np.int32)
        n = np.array([nopt[i] for i in sel], np.int32)
        ql = np.array([len(qids[i]) for i in sel], np.int32)
        ids = np.concatenate([qids[i] for i in sel]).astype(np.int32)
        t = np.ones(len(sel), np.float64)
        pr = np.zeros(int(n.sum()), np.float64)
        ch = np.zeros(len(sel), np.int32)
        cf = np.zeros(len(sel), np.float64)
        va = np.zeros(len(sel), np.float64)
        check(lib.dn_evaluate(h, len(sel), vp(k), vp(n), vp(ql), vp(ids), vp(t), MASK_ID, 1, vp(pr), vp(ch), vp(cf),
                              vp(va)), h)
        return pr, ch

    def batched():
        return call(list(range(nq)))

    def serial():
        outs = [call([i]) for i in range(nq)]
        return np.concatenate([o[0] for o in outs]), np.concatenate([o[1] for o in outs])

    T = sum(len(q) for q in qids)
    log(f"systemone: {nq} questions, {T} tokens per call")
    for _ in range(args.warmup):
        batched()
        serial()
    tb, ts = [], []
    quiesce_host()
    for _ in range(args.steps):
        t0 = time.perf_counter()
        pb, cb = batched()
        tb.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        ps, cs = serial()
        ts.append(time.perf_counter() - t0)
    agree = float(np.mean(cb == cs))
    dp = float(np.max(np.abs(pb - ps)))
    mb, ms = float(np.median(tb)), float(np.median(ts))
    result = {
        "metric": SYSTEMONE_METRIC,
        "value": round(1.0 / mb, 3),
        "unit": "calls/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mb * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "data": "synthetic: random-init weights N(0,0.02) (numpy PCG64 seed 0); 24 packed questions "
                "[CLS] 16 instruction ids + 2030 state ids [SEP] ([MASK] option)*K [SEP] (decide_amd/synth.py)",
        "config": {"workload": "systemone: 24 questions (Choice K=4 x6+, Noul K=2, Score K=5; cfg4 order) over one "
                               "2048-token state", "questions": nq, "tokens_per_call": T, "precision": args.precision},
        "batched_ms_per_call_p50": round(mb * 1e3, 3),
        "serial_ms_per_call_p50": round(ms * 1e3, 3),
        "speedup_batched_vs_serial": round(ms / mb, 3),
        "batched_tokens_per_s": round(T / mb, 1),
        "answers_agree_batched_vs_serial": {"choice_equal": agree, "max_abs_dprob_rounded": dp},
    }
    if not args.no_cpu_baseline:
        import oracle

        threads = cpu_threads()
        oracle.set_workers(threads)
        model = oracle.OracleModel(cfg, weights)
        secs, done = 0.0, 0
        while secs < args.cpu_budget and done < nq:
            i = done
            t0 = time.perf_counter()
            oracle.evaluate_question(model, {0: "choice", 1: "score", 2: "noul"}[kinds[i]], nopt[i], qids[i], MASK_ID,
                                     True, 1.0)
            secs += time.perf_counter() - t0
            done += 1
        per_q = secs / done
        result["cpu_baseline"] = {"value": round(1.0 / (per_q * nq), 5), "unit": "calls/s", "cores": threads,
                                  "kind": "port",
                                  "sample": f"{done} of the call's {nq} questions, one oracle forward each "
                                            f"({secs:.1f} s), scaled to the whole call; C++ restatement of the "
                                            "reference Go AVX2 path (oracle/)"}
    eng.close()
    print(json.dumps(result), flush=True)
    return 0


TRAIN_METRIC = ("training tokens/sec: one AdamW step over 32 examples (micro-batches within the trainer's TokenBudget, "
                "%d tokens), ModernBERT-base, 1 MI355X")


def quiesce_host() -> None:
    """Before a timed region: a full collection now, and the objects of the
    set-up (torch, numpy, the weights) moved out of the collector's reach, so
    that a full pass over them (~30 ms on the GPU box's host) does not land
    inside the timed steps."""
    gc.collect()
    gc.freeze()


def train_batches(cfg, n_examples=32, token_budget=4000, seed=0):
    """The trainer's step shape (internal/train/trainer.go:61-90, :270-330):
    BatchExamples 32 examples per optimizer step, packed to MaxLen 384
    (256-token premise + 8 options x 16), micro-batches of whole examples
    within TokenBudget (4000 by default on a GPU); one-hot targets."""
    from decide_amd.nn import MASK_ID, build_sequence
    from decide_amd.synth import pack_request

    rng = np.random.default_rng(2000 + seed)
    ex = [build_sequence(pack_request(rng, 256, [16] * 8, cfg.vocab), MASK_ID, True) for _ in range(n_examples)]
    targets = [np.eye(8)[int(rng.integers(0, 8))] for _ in range(n_examples)]
    per_micro = max(1, token_budget // 384)
    micro = [(ex[i:i + per_micro], targets[i:i + per_micro]) for i in range(0, n_examples, per_micro)]
    return ex, micro


def train_bench(args) -> int:
    """Times one optimizer step of the trainer's loop on the device
    (trainer.go:290-330): per micro-batch dn_forward_train, the soft
    cross-entropy on the host, dn_backward; then the gradient norm, clipping,
    dn_adamw_step and dn_zero_grad. Prints one JSON line."""
    import torch

    from decide_amd import modernbert_base
    from decide_amd.synth import random_weights
    from decide_amd.train import TrainEngine, soft_cross_entropy

    cfg = modernbert_base()
    log("generating weights")
    weights = random_weights(cfg, seed=0)
    ex, micro = train_batches(cfg, token_budget=args.token_budget)
    T = sum(len(s.ids) for s in ex)
    log(f"train: {len(ex)} examples, {T} tokens per step, {len(micro)} micro-batches")
    torch.cuda.init()
    eng = TrainEngine(cfg, weights, precision=args.precision, train_from=0, train_emb=False)
    n_items = len(ex)

    phases = {"forward": 0.0, "backward": 0.0, "update": 0.0}

    def step(timed=False):
        loss = 0.0
        for batch, targets in micro:
            t0 = time.perf_counter()
            logits = eng.forward(batch)
            t1 = time.perf_counter()
            l, dl = soft_cross_entropy(logits, targets, n_items)
            loss += l
            eng.backward(dl)
            t2 = time.perf_counter()
            if timed:
                phases["forward"] += t1 - t0
                phases["backward"] += t2 - t1
        t0 = time.perf_counter()
        gn = eng.grad_norm()
        scale = 1.0 if gn <= 1.0 else 1.0 / (gn + 1e-6)
        eng.update(4e-5, 3e-4, 0.01, scale)
        eng.zero_grad()
        if timed:
            phases["update"] += time.perf_counter() - t0
        return loss / n_items

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    log(f"timing {args.steps} steps")
    quiesce_host()
    eng.set_probe(1)
    losses, per_step = [], []
    for _ in range(args.steps):
        t0 = time.perf_counter()
        losses.append(step(timed=True))
        per_step.append(time.perf_counter() - t0)
    wall = sum(per_step)
    probe, nprobe = eng.read_probe_backward()
    eng.set_probe(-1)
    # Roofline kernel: layer 1's QKV weight-gradient GEMM (dWqkv += dqkv^T . n1,
    # 2 * 2304 * 768 flop per token; 2304 x 768 output in 64 x 192 tiles, run
    # unsplit over the tokens), timed with HIP events on
    # the weight-gradient stream; it shares the GPU with the main stream's
    # kernels while it runs.
    qkv_flop = 2.0 * (3 * H) * H * sum(len(s.ids) for s in ex) * args.steps
    wg_s = probe["wgrad_qkv"] * 1e-3
    dg_s = probe["dgrad_qkv"] * 1e-3
    log("backward probe ms per launch (layer 1): %s" % {k: round(v / max(nprobe, 1), 4) for k, v in probe.items()})
    result = {
        "metric": TRAIN_METRIC % args.token_budget,
        "value": round(T * args.steps / wall, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "data": "synthetic: random-init weights N(0,0.02) (numpy PCG64 seed 0), 32 packed examples "
                "[CLS] 254 ids [SEP] ([MASK] 15 ids)x8, one-hot targets (bench.py train_batches)",
        "config": {"workload": "train: 32 examples x 384 tokens per AdamW step, micro-batches of %d examples "
                               "(TokenBudget %d), all 22 layers trainable, embeddings frozen (trainer defaults)"
                               % (len(micro[0][0]), args.token_budget),
                   "examples_per_step": len(ex), "tokens_per_step": T, "micro_batches": len(micro),
                   "token_budget": args.token_budget, "precision": args.precision},
        "phase_ms_per_step": {k: round(v * 1e3 / args.steps, 3) for k, v in phases.items()},
        "loss_first_last": [round(losses[0], 5), round(losses[-1], 5)],
        "backward_probe_ms_per_launch": {k: round(v / max(nprobe, 1), 5) for k, v in probe.items()},
        "dgrad_qkv_tflops": round(qkv_flop / dg_s / 1e12, 2) if dg_s > 0 else None,
        "roofline": {"kernel": "gemm_nt_kernel<bf16,64,192,128,4,EPI_F32> accumulating into the gradient (one "
                               "split: 144 tiles): layer 1 dWqkv (weight-gradient stream, concurrent with the main "
                               "stream)",
                     "bound": "mfma", "achieved": round(qkv_flop / wg_s / 1e12, 2) if wg_s > 0 else None,
                     "peak": PEAK[args.precision] / 1e12, "unit": "TFLOP/s",
                     "frac": round(qkv_flop / wg_s / PEAK[args.precision], 4) if wg_s > 0 else None,
                     "traffic": None, "flop_per_step": qkv_flop / args.steps},
    }
    if not args.no_cpu_baseline:
        import oracle

        log("cpu baseline")
        threads = cpu_threads()
        oracle.set_workers(threads)
        model = oracle.OracleModel(cfg, weights)
        secs, toks, done = 0.0, 0, 0
        while secs < args.cpu_budget and done < len(ex):
            s = ex[done]
            t0 = time.perf_counter()
            logits = model.forward_train([s], 0)
            _, dl = soft_cross_entropy(logits, [micro[0][1][0]], 1)
            g = model.zeros_like()
            model.backward(dl, g, train_emb=False)
            secs += time.perf_counter() - t0
            toks += len(s.ids)
            done += 1
        result["cpu_baseline"] = {"value": round(toks / secs, 2), "unit": "tokens/s", "cores": threads,
                                  "kind": "port",
                                  "sample": f"{done} example(s) of 384 tokens, training forward + backward each "
                                            f"({secs:.1f} s; the optimizer step is not included); C++ restatement "
                                            "of the reference Go path (oracle/)"}
    eng.close()
    print(json.dumps(result), flush=True)
    return 0


def synthetic_prose(seed: int, n_docs: int, doc_words: int):
    """Pseudo-English documents: syllable words, capitals, digits,
    punctuation, contractions, some accented words and line breaks."""
    import random

    rng = random.Random(seed)
    syl = ["ta", "ke", "ri", "on", "mar", "sel", "ing", "pre", "con", "tion", "ab", "ly", "de", "ver", "st", "ou",
           "fi", "na", "lo", "gu", "ment", "er", "qu", "ist", "re", "ca", "pol", "ex", "un", "im"]
    extra = ["don't", "it's", "we're", "café", "naïve", "2026", "1,234.56", "(approx.)", "e.g.", "--", "%"]
    docs = []
    for _ in range(n_docs):
        words = []
        for i in range(doc_words):
            if rng.random() < 0.05:
                w = rng.choice(extra)
            else:
                w = "".join(rng.choice(syl) for _ in range(rng.randint(1, 4)))
                if rng.random() < 0.1:
                    w = w.capitalize()
            words.append(w + (rng.choice([",", ".", ":", "?"]) if rng.random() < 0.08 else ""))
            if rng.random() < 0.02:
                words.append("\n")
        docs.append(" ".join(words))
    return docs


def tokenizer_bench(args) -> int:
    """Host tokenizer throughput (dn_tokenize, one thread) on a byte-level BPE
    vocabulary of 8000 trained here, against HuggingFace `tokenizers` (one
    thread) and the oracle's pure-Python restatement. Prints one JSON line."""
    os.environ["TOKENIZERS_PARALLELISM"] = "false"
    from tokenizers import AddedToken, Tokenizer as HFTokenizer, models, normalizers, pre_tokenizers, processors, \
        trainers

    import oracle.tokenizer as ot
    from decide_amd.tokenizer import Tokenizer

    hf = HFTokenizer(models.BPE())
    hf.normalizer = normalizers.NFC()
    hf.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    hf.train_from_iterator(synthetic_prose(1, 4000, 200), trainers.BpeTrainer(
        vocab_size=8000, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(), show_progress=False))
    hf.add_special_tokens([AddedToken(t, special=True, normalized=False, lstrip=(t == "[MASK]"))
                           for t in ("[CLS]", "[SEP]", "[MASK]", "[PAD]", "[UNK]")])
    hf.post_processor = processors.TemplateProcessing(
        single="[CLS] $A [SEP]", special_tokens=[("[CLS]", hf.token_to_id("[CLS]")), ("[SEP]", hf.token_to_id("[SEP]"))])
    raw = hf.to_str().encode()
    tok = Tokenizer.parse(raw)
    docs = synthetic_prose(2, 400, 400)
    nbytes = sum(len(d.encode()) for d in docs)

    def timed(fn, budget):
        n_tok, secs, k = 0, 0.0, 0
        while secs < budget:
            d = docs[k % len(docs)]
            t0 = time.perf_counter()
            n_tok += len(fn(d))
            secs += time.perf_counter() - t0
            k += 1
        return n_tok / secs, k, secs

    for d in docs:  # warm the word caches once (both implementations keep one)
        tok.encode(d)
        hf.encode(d)
    lib_tps, lib_docs, lib_s = timed(tok.encode, 3.0)
    hf_tps, _, _ = timed(lambda d: hf.encode(d).ids, 3.0)
    orc = ot.Tokenizer(raw)
    orc_tps, orc_docs, orc_s = timed(orc.encode, args.cpu_budget / 2)
    same = all(tok.encode(d) == hf.encode(d).ids for d in docs[:50])
    avg_bytes_per_tok = nbytes / sum(len(tok.encode(d)) for d in docs)
    result = {
        "metric": "host tokenizer throughput: byte-level BPE (NFC, GPT-2 pre-tokenizer), vocab 8000, one thread",
        "value": round(lib_tps, 1),
        "unit": "tokens/s",
        "n_gpus": 0,
        "steps": lib_docs,
        "warmup": len(docs),
        "ms_per_step": round(lib_s * 1e3 / lib_docs, 4),
        "higher_is_better": True,
        "scaling": "strong",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic pseudo-English documents of 400 words (bench.py synthetic_prose), vocabulary trained "
                "here with HuggingFace tokenizers",
        "config": {"workload": "tokenize 400 documents (%d bytes) one at a time" % nbytes, "vocab": 8000},
        "mb_per_s": round(lib_tps * avg_bytes_per_tok / 1e6, 2),
        "huggingface_tokenizers_tokens_per_s": round(hf_tps, 1),
        "ids_equal_huggingface": same,
        "cpu_baseline": {"value": round(orc_tps, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
                         "sample": f"{orc_docs} documents, {orc_s:.1f} s; the oracle's pure-Python restatement of "
                                   "internal/tokenizer/tokenizer.go"},
    }
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--precision", default="bf16", choices=["bf16", "fp16", "fp32"])
    ap.add_argument("--certify", type=float, default=0.0, metavar="MARGIN",
                    help="dn_set_certify margin (16-bit precisions; 0: off)")
    ap.add_argument("--nseq", type=int, default=None,
                    help="sequences of the configuration's shape (default: the configuration's batch)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--probe-layer", type=int, default=1)
    ap.add_argument("--probe-steps", type=int, default=5,
                    help="forwards run with the per-launch probe after the timed ones (one stream)")
    ap.add_argument("--stream-split", type=int, default=8192, metavar="TOKENS",
                    help="dn_set_stream_split: batches of at least TOKENS run in two parts on two streams (0: off)")
    ap.add_argument("--row-tail", type=int, default=2048, metavar="TOKENS",
                    help="dn_set_row_tail: batches of at least TOKENS finish the last layer on the option rows (0: off)")
    ap.add_argument("--ln-fold", type=int, default=1, choices=(0, 1),
                    help="dn_set_ln_fold: bf16 and fp16 batches of more than 1024 tokens run the LayerNorms inside the GEMMs")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run one device copy of MIB MiB first (reference kernel for HBM counters)")
    ap.add_argument("--tokenizer", action="store_true",
                    help="time the host tokenizer (dn_tokenize) against HuggingFace tokenizers; no GPU")
    ap.add_argument("--library-gemm", action="store_true",
                    help="time the projection GEMM shapes alone: this library's kernels vs hipBLASLt (torch.mm)")
    ap.add_argument("--systemone", action="store_true",
                    help="time one SystemOne call (24 questions) batched into one forward vs one forward each")
    ap.add_argument("--train", action="store_true",
                    help="time one training step (forward, backward, AdamW) at the trainer's GPU shape")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="default run: skip the cfg1 / cfg2 / cfg4 / cfg5 measurements after the headline")
    ap.add_argument("--summarize-traffic", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "OUT_JSON"),
                    help="write the HBM traffic summary of two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE)")
    ap.add_argument("--token-budget", type=int, default=4000,
                    help="--train: tokens per micro-batch (the trainer's TokenBudget; 4000 is its GPU default)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the forward shards by sequence with no collective on the hot path)", file=sys.stderr)
        return 2

    if args.summarize_traffic:
        return summarize_traffic(*args.summarize_traffic)
    if args.tokenizer:
        return tokenizer_bench(args)
    if args.systemone:
        return systemone(args)
    if args.library_gemm:
        return library_gemm(args)
    if args.train:
        return train_bench(args)

    import torch

    from decide_amd import Engine, modernbert_base
    from decide_amd.synth import random_weights

    cfg = modernbert_base()
    log("generating weights")
    weights = random_weights(cfg, seed=0)
    torch.cuda.init()
    dev = torch.device("cuda:0")
    eng = Engine(cfg, weights, precision=args.precision, certify=args.certify)
    stream = torch.cuda.current_stream()
    eng.set_stream(stream.cuda_stream)

    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {nbytes} bytes read + {nbytes} bytes written")
        del src, dst

    eng.set_stream_split(args.stream_split)
    eng.set_row_tail(args.row_tail)
    eng.set_ln_fold(bool(args.ln_fold))
    wl = Workload(eng, cfg, args.config, dev, nseq=args.nseq)
    log(f"workload {args.config}: {wl.nseq} sequences, T={wl.T}, R={wl.R}")
    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()
    eng.check_device_errors()
    eng.read_certify()  # counters cover the timed steps only

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    log(f"timing {args.steps} steps")
    quiesce_host()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for k in range(args.steps):
        wl.step()
        ev[k + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    eng.check_device_errors()
    cert_counts = eng.read_certify()
    # Per-launch kernel durations: a separate run with the probe on (HIP
    # events around layer probe_layer's five launches), where forwards run on
    # one stream so that each interval times one kernel alone.
    eng.set_probe(args.probe_layer)
    for _ in range(args.probe_steps):
        wl.step()
    probe, nprobe = eng.read_probe()
    eng.set_probe(-1)
    per_step = [ev[k].elapsed_time(ev[k + 1]) for k in range(args.steps)]
    gpu_ms = sum(per_step)
    T = wl.T
    value = T * args.steps / wall
    avg = {k: v / max(nprobe, 1) for k, v in probe.items()}
    log("per-launch ms (layer %d): %s" % (args.probe_layer, {k: round(v, 4) for k, v in avg.items()}))

    prec = args.precision
    esz = 4 if prec == "fp32" else 2
    tname = {"bf16": "bf16", "fp16": "f16", "fp32": "float"}[prec]
    hbm_bound = T <= 128
    attain = None
    if prec != "fp32":
        m0 = 0 if prec == "bf16" else 4
        attain = {"changing_operands_tflops": round(eng.mfma_calibrate(m0), 1),
                  "constant_operands_tflops": round(eng.mfma_calibrate(m0 + 1), 1),
                  "method": f"dn_mfma_calibrate: register-only v_mfma_f32_32x32x16_{tname} loop in the GEMMs' wave "
                            "pattern on every CU, 2 waves per SIMD, no memory traffic; operands N(0,1) x "
                            "N(0,0.02), rotated one lane per iteration (changing) or fixed (constant)"}
        if prec == "fp16":
            attain["bf16_changing_operands_tflops"] = round(eng.mfma_calibrate(0), 1)
    # Per-launch roofline views. The kernel with the largest share of GPU
    # time at cfg3 is the fp32-residual GEMM (Wo and MlpWo share its symbol):
    # algorithmic bytes per launch are A, the weights, and the fp32 residual
    # read and written (T x H each way); with the folded LayerNorm (16-bit,
    # T > 1024) also the next norm's 16-bit operand (T x H) and the row
    # statistics (8 bytes per row and 192 columns) it writes. By the roofline
    # model it is bound by HBM (its bytes take longer at 8 TB/s than its flops
    # at the MFMA peak).
    fold = bool(args.ln_fold) and prec in ("bf16", "fp16") and T > 1024
    res_s = (avg["gemm_wo"] + avg["gemm_mlpwo"]) * 1e-3
    res_bytes = esz * (T * H + H * H) + esz * (T * I + H * I) + 2 * 2 * 4 * T * H
    if fold:
        res_bytes += 2 * (esz * T * H + 8 * T * (H // 192))
    res_flop = 2.0 * T * H * (H + I)
    wi_flop = 2.0 * T * (2 * I) * H
    wi_bytes = esz * (T * H + 2 * I * H + T * I)
    wi_s = avg["gemm_wi"] * 1e-3
    traffic = read_traffic(args.config, prec, fold)
    res_name = (f"gemm_nt_kernel<{tname},256,192,128,2,EPI_F32_LN,2,4,2> (Wo and MlpWo + fp32 residual + the next "
                "LayerNorm's operand and statistics)" if fold else
                f"gemm_nt_kernel<{tname},256,192,128,2,EPI_F32,2,4,2> (Wo and MlpWo + fp32 residual)")
    if hbm_bound:
        # small M (cfg2, cfg5): the skinny kernel streams the weights; the Wi
        # launch (the largest weight matrix) is the line
        roof = {"kernel": "gemm_skinny_kernel, EPI_GEGLU (Wi projection + fused GeGLU), layer %d" % args.probe_layer,
                "bound": "hbm", "achieved": round(wi_bytes / wi_s / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(wi_bytes / wi_s / 8e12, 4), "traffic": None,
                "algorithmic_bytes_per_launch": wi_bytes}
    else:
        roof = {"kernel": res_name + ", layer %d, average of its two launches" % args.probe_layer,
                "bound": "hbm", "achieved": round(res_bytes / res_s / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(res_bytes / res_s / 8e12, 4), "traffic": traffic.get("residual"),
                "algorithmic_bytes_per_launch": res_bytes / 2,
                "mfma_view": {"achieved_tflops": round(res_flop / res_s / 1e12, 2),
                              "frac_of_2500": round(res_flop / res_s / PEAK[prec], 4),
                              "flop_per_launch": res_flop / 2}}
    gemm_ms = avg["gemm_qkv"] + avg["gemm_wo"] + avg["gemm_wi"] + avg["gemm_mlpwo"]
    gemm_tflops = PROJ_FLOP_PER_TOKEN_LAYER * T / (gemm_ms * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": prec,
        "data": "synthetic: random-init weights N(0,0.02) (InitRandom semantics, numpy PCG64 seed 0), "
                "token ids uniform in [5,50368) minus specials, packed [CLS] premise [SEP] ([MASK] option)xK",
        "config": {"workload": WORKLOADS[args.config], "batch": wl.nseq, "seq_len": wl.max_len,
                   "tokens_per_step": T, "rows_per_step": wl.R, "layers": cfg.layers, "precision": prec,
                   "timed_call": "dn_forward_device (token arrays resident on the device)"},
        "gpu_ms_per_step_events": round(gpu_ms / args.steps, 4),
        "step_ms_p50": round(float(np.percentile(per_step, 50)), 4),
        "step_ms_p99": round(float(np.percentile(per_step, 99)), 4),
        "projection_gemm_tflops": round(gemm_tflops, 2),
        "projection_gemm_frac_peak": round(gemm_tflops * 1e12 / PEAK[prec], 4),
        "per_launch_ms": {k: round(v, 5) for k, v in avg.items()},
        "per_launch_method": f"HIP events on the launch stream around layer {args.probe_layer}'s launches, "
                             f"{nprobe} forwards run after the timed ones on one stream",
        "stream_split_min_tokens": args.stream_split,
        "row_tail_min_tokens": args.row_tail,
        "ln_fold": bool(args.ln_fold),
        "roofline": roof,
    }
    if args.certify:
        result["certify"] = {"margin": args.certify,
                             "sequences_checked": cert_counts[0], "sequences_recomputed_fp32": cert_counts[1],
                             "method": "dn_set_certify: sequences whose two best logits are closer than the margin "
                                       "are recomputed on the fp32 twin inside each timed step"}
    if attain:
        result["mfma_attainable"] = attain
        result["projection_gemm_frac_attainable"] = round(gemm_tflops / attain["changing_operands_tflops"], 4)
    if not hbm_bound:
        result["roofline_wi_gemm"] = {
            "kernel": f"gemm_nt_kernel<{tname},256,128,64,3,{'EPI_GEGLU_LN' if fold else 'EPI_GEGLU'},2,2,2> "
                      f"(Wi projection + fused GeGLU{' + folded mlp_norm' if fold else ''}), layer %d"
                      % args.probe_layer,
            "bound": "mfma", "achieved": round(wi_flop / wi_s / 1e12, 2), "peak": PEAK[prec] / 1e12,
            "unit": "TFLOP/s", "frac": round(wi_flop / wi_s / PEAK[prec], 4), "traffic": traffic.get("wi"),
            "flop_per_launch": wi_flop, "algorithmic_bytes_per_launch": wi_bytes}
    # The same workload through the host-array entry point (ids/pos/opt in,
    # logits out; PCIe copies included): never the headline value.
    hio = []
    for _ in range(max(3, args.steps // 4)):
        t1 = time.perf_counter()
        wl.host_forward()
        hio.append(time.perf_counter() - t1)
    result["host_io_tokens_per_s"] = round(T / float(np.median(hio)), 1)
    if not args.no_extra_configs and args.config == "cfg3" and prec != "fp32":
        result["configs"] = extra_configs(eng, cfg, dev, stream, args)
    if not args.no_extra_configs and prec == "bf16" and not args.certify:
        eng.close()
        eng = None
        result["certified_fp16"] = certified_run(cfg, weights, dev, stream, args)
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(cfg, weights, args.config, args.cpu_budget)
        result["cpu_baseline_1thread"] = cpu_baseline(cfg, weights, args.config, args.cpu_budget, threads=1)
        result["host_cpu"] = host_cpu_info()
        if "configs" in result:
            result["configs"]["cfg1"]["oracle_sgemm"] = [cpu_gemm_cfg1(cpu_threads()), cpu_gemm_cfg1(1)]
    if eng is not None:
        eng.close()
    print(json.dumps(result), flush=True)
    return 0


def certified_run(cfg, weights, dev, stream, args, margin=1e-3) -> dict:
    """The same workload with the answers certified against the reference
    (fp16 operands + dn_set_certify: sequences whose two best logits are
    closer than `margin`, ~8x the fp16 path's RMS error of a logit difference,
    are recomputed on the fp32 twin inside the step), and the latency of one
    cfg2 / cfg5 request through dn_forward in that mode."""
    import torch

    from decide_amd import Engine

    eng = Engine(cfg, weights, precision="fp16", certify=margin)
    eng.set_stream(stream.cuda_stream)
    eng.set_stream_split(args.stream_split)
    eng.set_row_tail(args.row_tail)
    wl = Workload(eng, cfg, args.config, dev, nseq=args.nseq)
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()
    eng.read_certify()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        wl.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    checked, recomputed = eng.read_certify()
    out = {"precision": "fp16", "certify_margin": margin, "tokens_per_s": round(wl.T * args.steps / wall, 1),
           "ms_per_step": round(wall * 1e3 / args.steps, 4), "sequences_checked": checked,
           "sequences_recomputed_fp32": recomputed,
           "timed_call": "dn_forward_device with dn_set_certify (synchronous: logits read back, near-ties "
                         "recomputed on the fp32 twin, logits written back)"}
    for name, reps in (("cfg2", 500), ("cfg5", 2000)):
        w2 = Workload(eng, cfg, name, dev)
        for _ in range(20):
            w2.host_forward()
        eng.read_certify()
        lat = np.empty(reps)
        for r in range(reps):
            t1 = time.perf_counter()
            w2.host_forward()
            lat[r] = time.perf_counter() - t1
        _, rc = eng.read_certify()
        out[name] = {"latency_ms_p50": round(float(np.percentile(lat, 50)) * 1e3, 4),
                     "latency_ms_p99": round(float(np.percentile(lat, 99)) * 1e3, 4),
                     "requests": reps, "recomputed": rc}
    eng.close()
    return out


class Workload:
    """One configuration's batch, staged on the device for dn_forward_device."""

    def __init__(self, eng, cfg, name, dev, nseq=None):
        import torch

        from decide_amd.nn import flatten, row_tokens
        from decide_amd.synth import config_batch

        self.eng, self.batch = eng, config_batch(name, vocab=cfg.vocab, nseq=nseq)
        self.seq_len, ids, pos, opt, nmask, _ = flatten(self.batch)
        self.T, self.R, self.nseq = int(self.seq_len.sum()), int(nmask.sum()), len(self.batch)
        self.max_len = int(self.seq_len.max())
        self.d_ids = torch.from_numpy(ids).to(dev)
        self.d_pos = torch.from_numpy(pos).to(dev)
        self.d_opt = torch.from_numpy(opt).to(dev)
        self.d_rt = torch.from_numpy(row_tokens(self.batch)).to(dev)
        self.d_out = torch.zeros(self.R, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()

    def step(self):
        self.eng.forward_device(self.seq_len, self.d_ids.data_ptr(), self.d_pos.data_ptr(), self.d_opt.data_ptr(),
                                self.R, self.d_rt.data_ptr(), self.d_out.data_ptr())

    def host_forward(self):
        return self.eng.forward(self.batch)


def extra_configs(eng, cfg, dev, stream, args) -> dict:
    """The other BASELINE configurations on the same engine and weights:
    cfg1 (the fp32 projection GEMM on fp32 MFMA), cfg2 and cfg5 (one request:
    latency of the host-array dn_forward call, and achieved weight-streaming
    GB/s), cfg4 (8 x 2816-token SystemOne sequences: tokens/s)."""
    import torch

    out = {}
    # cfg1: X[512x768] . W^T, W[2304x768], fp32 operands resident on the device
    M, N, K = 512, 2304, 768
    g = torch.Generator().manual_seed(0)
    dA = torch.randn(M, K, generator=g).to(dev)
    dB = (torch.randn(N, K, generator=g) * 0.02).to(dev)
    dC = torch.zeros(M, N, device=dev)
    for _ in range(5):
        eng.gemm_device("fp32", M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 200
    e0.record(stream)
    for _ in range(reps):
        eng.gemm_device("fp32", M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr())
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    flop = 2.0 * M * N * K
    out["cfg1"] = {"workload": "fp32 X[512x768] . W^T, W[2304x768] on fp32 MFMA (dn_gemm_device, operands resident)",
                   "us_per_call": round(us, 2), "tflops": round(flop / us / 1e6, 2),
                   "frac_of_fp32_peak": round(flop / us / 1e6 / 157.3, 4)}
    # the fp32 matrix cores' attainable rate on such operands (register-only loop)
    att32 = eng.mfma_calibrate(2)
    out["cfg1"]["fp32_mfma_attainable_tflops"] = round(att32, 1)
    out["cfg1"]["frac_of_fp32_attainable"] = round(flop / us / 1e6 / att32, 4) if att32 > 0 else None
    # cfg2 and cfg5: latency of one request through the host-array entry point
    for name, reps in (("cfg2", 1000), ("cfg5", 10000)):
        wl = Workload(eng, cfg, name, dev)
        for _ in range(20):
            wl.host_forward()
        lat = np.empty(reps)
        for r in range(reps):
            t1 = time.perf_counter()
            wl.host_forward()
            lat[r] = time.perf_counter() - t1
        # device time per forward (events around back-to-back device forwards)
        e0.record(stream)
        for _ in range(200):
            wl.step()
        e1.record(stream)
        torch.cuda.synchronize()
        dev_ms = e0.elapsed_time(e1) / 200
        # The same forward right after a 1 GiB device copy has swept the last-level cache (MALL,
        # 256 MB, which can hold most of the 220.6 MB of weights between back-to-back forwards):
        # whether that residency flatters dev_ms. The copy runs on the launch stream before the
        # timed forward.
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        cold = []
        for _ in range(20):
            dst.copy_(src)
            e0.record(stream)
            wl.step()
            e1.record(stream)
            torch.cuda.synchronize()
            cold.append(e0.elapsed_time(e1))
        del src, dst
        wbytes = 2 * cfg.layers * H * (3 * H + H + 2 * I + I)  # bf16 projection weights streamed per forward
        out[name] = {"workload": WORKLOADS[name], "repetitions": reps,
                     "latency_ms_p50": round(float(np.percentile(lat, 50)) * 1e3, 4),
                     "latency_ms_p99": round(float(np.percentile(lat, 99)) * 1e3, 4),
                     "latency_call": "dn_forward (host ids in, logits out), wall clock per call",
                     "device_ms_per_forward": round(dev_ms, 4),
                     "tokens_per_s": round(wl.T / (dev_ms * 1e-3), 1),
                     "weight_bytes_per_forward": wbytes,
                     "achieved_GBps": round(wbytes / (dev_ms * 1e-3) / 1e9, 1),
                     "frac_of_8TBps": round(wbytes / (dev_ms * 1e-3) / 8e12, 4),
                     "device_ms_per_forward_cache_swept": round(float(np.median(cold)), 4)}
    # cfg4: 8 sequences of 2816 tokens
    wl = Workload(eng, cfg, "cfg4", dev)
    for _ in range(3):
        wl.step()
    e0.record(stream)
    steps = 10
    for _ in range(steps):
        wl.step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    eng.check_device_errors()
    out["cfg4"] = {"workload": WORKLOADS["cfg4"], "ms_per_forward": round(ms, 4),
                   "tokens_per_s": round(wl.T / (ms * 1e-3), 1)}
    return out


# Template arguments <BM, BN, BK, STAGES, EPI, WG/CU, wave rows, wave cols>
# of the 16-bit roofline kernels at cfg3 (launch_gemm16's choice for T =
# 32768): the residual GEMMs (N = 768) and the Wi GEMM (N = 2 x 1152).
ROOF_TILES = {"residual": [256, 192, 128, 2, 0, 2, 4, 2], "wi": [256, 128, 64, 3, 2, 2, 2, 2],
              "qkv": [256, 128, 64, 3, 1, 2, 2, 2]}
# With the folded LayerNorm (the default 16-bit forward above 1024 tokens) the
# same tiles run the EPI_F32_LN / EPI_GEGLU_LN / EPI_STORE_LN epilogues.
FOLD_EPI = {"residual": 5, "wi": 7, "qkv": 6}


def roof_tiles(fold: bool) -> dict:
    if not fold:
        return ROOF_TILES
    return {k: v[:4] + [FOLD_EPI[k]] + v[5:] for k, v in ROOF_TILES.items()}


def read_traffic(config: str, prec: str, fold: bool = False) -> dict:
    """HBM bytes per launch of the roofline kernels, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/), when it covers
    this workload."""
    path = os.path.join(HERE, "profiles", "gemm_traffic_cfg3.json")
    if config != "cfg3" or prec != "bf16" or not os.path.exists(path):
        return {}
    with open(path) as fh:
        d = json.load(fh)
    # A summary of other tile shapes than the ones launched now describes
    # another kernel: its bytes are not reported.
    tiles = roof_tiles(fold)
    return {k: v.get("hbm_bytes_per_launch") for k, v in d.get("kernels", {}).items()
            if v.get("template_args") == tiles.get(k)}


def summarize_traffic(fetch_dir: str, write_dir: str, out_path: str) -> int:
    """Turns two rocprofv3 --pmc runs of `bench.py --steps 2 --warmup 1
    --probe-steps 1 --no-cpu-baseline --no-extra-configs --copy-calibration 512
    --stream-split 0` (FETCH_SIZE, then WRITE_SIZE; one stream, so every GEMM
    launch covers the whole batch) into bytes per launch for the roofline
    kernels, each counter scaled by what it reads for the 512 MiB device
    copy."""
    import csv
    import glob

    def per_dispatch(d, counter):
        acc, names = {}, {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                key = (f, r["Dispatch_Id"])  # rows of one dispatch (per XCD where split) are summed
                acc[key] = acc.get(key, 0.0) + float(r["Counter_Value"]) * 1024.0
                names[key] = r["Kernel_Name"]
        byk = {}
        for key, v in acc.items():
            byk.setdefault(names[key], []).append(v)
        return byk

    def gemm_params(name):
        """Template arguments of gemm_nt_kernel<bf16, BM, BN, BK, STAGES, EPI, ...>
        (or gemm_nt_ln_kernel, the folded-LayerNorm forms) from a mangled
        (..Li128ELi192E..) or demangled (<.., 128, 192, ..>) name."""
        kind = "gemm_nt_ln_kernel" if "gemm_nt_ln_kernel" in name else "gemm_nt_kernel"
        if kind not in name:
            return None
        tail = name.split(kind, 1)[1]
        m = re.findall(r"Li(\d+)E", tail)
        if not m:
            m = re.findall(r"(?<=[<,\s])(\d+)(?=[,>])", tail.split(">")[0] + ">")
        return tuple(int(x) for x in m)

    fetch, write = per_dispatch(fetch_dir, "FETCH_SIZE"), per_dispatch(write_dir, "WRITE_SIZE")
    copy_bytes = 512 << 20
    # The calibration copy is the largest copy dispatch of each run.
    fetch_scale = copy_bytes / max(max(v) for k, v in fetch.items() if "copyBuffer" in k)
    write_scale = copy_bytes / max(max(v) for k, v in write.items() if "copyBuffer" in k)
    T = 32768
    alg = {"residual": (2 * (T * H + H * H) + 2 * (T * I + H * I) + 16 * T * H) / 2,
           "wi": 2 * (T * H + 2 * I * H + T * I), "qkv": 2 * (T * H + 3 * H * H + 3 * T * H)}
    # The folded-LayerNorm forms (when the run launched them): the residual
    # GEMM also writes the bf16 operand and 8 bytes of statistics per row
    # and 192 columns; QKV and Wi read those statistics and a row mean and
    # write a row mean (40 bytes per row).
    alg_fold = {"residual": alg["residual"] + 2 * T * H + 8 * T * (H // 192),
                "wi": alg["wi"] + 40 * T, "qkv": alg["qkv"] + 40 * T}
    kernels = {}
    for name in ROOF_TILES:
        cands, fold = [], False
        for fold in (True, False):
            tiles = roof_tiles(fold)[name]
            cands = [k for k in fetch if list(gemm_params(k) or ())[:5] == tiles[:5]]
            if cands:
                break
        if not cands:
            continue
        k = cands[0]
        fb = float(np.mean(fetch[k])) * fetch_scale
        wb = float(np.mean(write.get(k, [0.0]))) * write_scale
        kernels[name] = {"symbol": k, "template_args": list(gemm_params(k)), "dispatches": len(fetch[k]),
                         "fetch_bytes_per_launch": round(fb), "write_bytes_per_launch": round(wb),
                         "hbm_bytes_per_launch": round(fb + wb),
                         "algorithmic_bytes_per_launch": (alg_fold if fold else alg)[name],
                         "traffic_over_algorithmic": round((fb + wb) / (alg_fold if fold else alg)[name], 3)}
    others = {}
    for k, v in fetch.items():
        if "attention_kernel" in k or ("ln_kernel" in k and "gemm_nt_ln_kernel" not in k):
            # Per symbol; the summary keeps each family's most-dispatched
            # variant (attention: the full-batch layers, not the last layer's
            # row-tail variant).
            tag = "attention" if "attention_kernel" in k else "layernorm"
            if tag in others and others[tag]["dispatches"] >= len(v):
                continue
            others[tag] = {"symbol": k, "dispatches": len(v),
                           "fetch_bytes_per_launch": round(float(np.mean(v)) * fetch_scale),
                           "write_bytes_per_launch": round(float(np.mean(write.get(k, [0.0]))) * write_scale)}
    res = {"workload": "cfg3 (T=32768), bf16", "fetch_scale": fetch_scale, "write_scale": write_scale,
           "method": "rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE (separate runs of bench.py --steps 2 "
                     "--warmup 1 --probe-steps 1 --no-cpu-baseline --no-extra-configs --copy-calibration 512 "
                     "--stream-split 0), KiB per dispatch "
                     "summed over XCDs and averaged over the dispatches of each symbol, scaled by the counter's "
                     "reading for the 512 MiB device copy (the largest copy dispatch of each run)", "kernels": kernels,
           "other_kernels": others}
    with open(out_path, "w") as fh:
        json.dump(res, fh, indent=1)
    print(json.dumps(res, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
