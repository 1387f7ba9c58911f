"""The reference-side binding as code: go/hipnn/hipnn.go (purego, as
internal/cuda loads libcuda) and go/hipnn/wiring.patch (NewInferer, Local).

There is no Go toolchain in this image, so what a Go build would check is
checked here: every symbol the binding registers is declared in
include/decide_hip.h and exported by libdecide_hip.so; each Go func type has
the C prototype's arity and argument kinds; and tests/abi_replay.c replays
the binding's call sequence through dlopen(RTLD_NOW | RTLD_GLOBAL) and dlsym
(internal/cuda/lib_unix.go:7-9, driver.go:62-105): Load -> New -> Forward ->
Free, with dn_open's DN_NO_GPU, a missing library and a missing symbol each
ending in ErrNoGPU as the binding maps them."""
import ctypes
import os
import re
import shutil
import struct
import subprocess

import numpy as np
import pytest

from conftest import ROOT

GO_SRC = os.path.join(ROOT, "go", "hipnn", "hipnn.go")
HEADER = os.path.join(ROOT, "include", "decide_hip.h")
LIB = os.environ.get("DECIDE_HIP_LIBRARY") or os.path.join(ROOT, "decide_amd", "libdecide_hip.so")


def go_bindings():
    """{symbol: (go param types, go result type)} from the api struct and the
    reg(&lib.field, "symbol") calls of hipnn.go."""
    src = open(GO_SRC).read()
    body = re.search(r"type api struct \{(.*?)\n\}", src, re.S).group(1)
    fields = {}
    for m in re.finditer(r"^\s*(\w+)\s+func\((.*?)\)\s*([\w*]*)\s*$", body, re.M):
        name, params, ret = m.groups()
        types, pending = [], 0
        for part in [p.strip() for p in params.split(",") if p.strip()]:
            words = part.split()
            if len(words) == 1:  # a name whose type comes later (a, b int32)
                pending += 1
                continue
            types += [words[-1]] * (pending + 1)
            pending = 0
        assert pending == 0, (name, params)
        fields[name] = (types, ret)
    regs = re.findall(r'reg\(&lib\.(\w+), "(\w+)"\)', src)
    assert regs and len({s for _, s in regs}) == len(regs)
    return {sym: fields[f] for f, sym in regs}


C_TO_GO = {"int": "int32", "int32_t": "int32", "int64_t": "int64", "float": "float32", "double": "float64",
           "dn_ctx*": "uintptr", "dn_ctx**": "*uintptr", "char*": "string", "uint8_t*": "*uint8",
           "int32_t*": "*int32", "float*": "*float32", "double*": "*float64", "void": ""}


def c_prototypes():
    """{symbol: (param types, result type)} of the header's extern "C" block,
    comments removed, const and parameter names dropped, pointers attached."""
    text = re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    protos = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(dn_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret, name, params = m.groups()

        def norm(decl, drop_name):
            decl = decl.replace("const", " ").replace("*", " * ")
            words = decl.split()
            if drop_name and len(words) > 1 and words[-1] != "*":
                words = words[:-1]
            base = [w for w in words if w != "*"]
            return base[-1] + "*" * words.count("*") if base else ""

        ps = [] if params.strip() in ("", "void") else [norm(p, True) for p in params.split(",")]
        protos[name] = (ps, norm(ret.split("\n")[-1], False))
    return protos


def test_binding_symbols_are_declared_and_exported():
    binds, protos = go_bindings(), c_prototypes()
    lib = ctypes.CDLL(LIB, mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    for sym in binds:
        assert sym in protos, f"{sym} is not declared in include/decide_hip.h"
        assert hasattr(lib, sym), f"{sym} is not exported by {LIB}"
    # the inference path's entry points are all there
    assert {"dn_open", "dn_set_config", "dn_upload_tensor", "dn_forward", "dn_close", "dn_evaluate"} <= set(binds)


def test_binding_types_match_the_c_prototypes():
    binds, protos = go_bindings(), c_prototypes()
    for sym, (go_params, go_ret) in binds.items():
        c_params, c_ret = protos[sym]
        want = [C_TO_GO[t] for t in c_params]
        assert go_params == want, (sym, go_params, want)
        assert go_ret == C_TO_GO[c_ret], (sym, go_ret, c_ret)


def test_wiring_patch_names_the_binding():
    """The patch hooks both inference entry points and keeps ErrNoGPU's
    fall-through (engine.go:42-61's pattern); it applies to the reference
    sources (checked with `patch -p1 --dry-run` where they are present)."""
    patch = open(os.path.join(ROOT, "go", "hipnn", "wiring.patch")).read()
    assert "+++ b/internal/train/engine.go" in patch and "+++ b/local.go" in patch
    assert patch.count("errors.Is(") >= 2 and "hipnn.ErrNoGPU" in patch
    assert "lm.dev.Forward([]nn.Sequence{seq})" in patch
    # Local.Evaluate answers a whole call with one batched hipnn.Evaluate,
    # per-question failures reported under the question's id
    assert "lm.dev.Evaluate(" in patch and "var qe *hipnn.QuestionError" in patch
    assert 'fmt.Errorf("decide: question %q: %w", id, err)' in patch
    assert "hipnn.NewWith(b.Model, hipnn.PrecisionFP16, hipnn.DefaultCertifyMargin)" in patch
    for name in re.findall(r"hipnn\.(\w+)\(", patch):
        assert re.search(rf"^func {name}\(", open(GO_SRC).read(), re.M), name
    ref = "/root/reference"
    if os.path.isdir(ref) and shutil.which("patch"):
        r = subprocess.run(["patch", "-p1", "--dry-run", "-i", os.path.join(ROOT, "go", "hipnn", "wiring.patch")],
                           cwd=ref, capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr


@pytest.fixture(scope="module")
def replay(tmp_path_factory):
    gcc = shutil.which("gcc") or shutil.which("cc")
    if not gcc:
        pytest.skip("no C compiler")
    d = tmp_path_factory.mktemp("replay")
    exe = str(d / "abi_replay")
    subprocess.run([gcc, "-O1", "-Wall", "-o", exe, os.path.join(ROOT, "tests", "abi_replay.c"), "-ldl"],
                   check=True)
    syms = d / "symbols.txt"
    syms.write_text("\n".join(go_bindings()) + "\n")

    def run(*args, lib=LIB, symbols=str(syms)):
        r = subprocess.run([exe, lib, symbols, *args], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stdout + r.stderr
        return r.stdout.splitlines()

    run.dir = d
    return run


def has_gpu():
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


def test_replay_load_and_no_gpu(replay):
    """Load resolves exactly the binding's symbols; on a machine without a
    GPU dn_open's DN_NO_GPU is ErrNoGPU (the CPU fallback of openDevice)."""
    out = replay()
    assert out[0] == f"resolved {len(go_bindings())} symbols"
    if has_gpu():
        assert out[1] == "opened and closed"
    else:
        assert out[1].startswith("ErrNoGPU (decide_hip: no GPU")


def test_replay_missing_library_or_symbol_is_no_gpu(replay):
    assert replay(lib=str(replay.dir / "libnot_there.so"))[0].startswith("ErrNoGPU (")
    bad = replay.dir / "bad_symbols.txt"
    bad.write_text("dn_open\ndn_forward_v2\n")
    assert replay(symbols=str(bad)) == ["ErrNoGPU (library is missing dn_forward_v2)"]


def write_manifest(path_m, path_w, cfg, weights, batch, precision):
    from decide_amd.nn import tensor_shapes

    lines = ["config %d %d %d %d %d %r %d %r %r %d %s" % (
        cfg.hidden, cfg.intermediate, cfg.heads, cfg.layers, cfg.vocab, float(np.float32(cfg.eps)),
        cfg.half_window, float(cfg.global_theta), float(cfg.local_theta), precision,
        " ".join("1" if s else "0" for s in cfg.sliding))]
    with open(path_w, "wb") as fw:
        for name, shape in tensor_shapes(cfg).items():
            a = np.ascontiguousarray(weights[name], np.float32).reshape(-1)
            fw.write(a.tobytes())
            lines.append(f"tensor {name} {a.size}")
    for s in batch:
        lines.append(f"seq {len(s.ids)} {0 if s.opt is None else 1} {len(s.mask_pos)}")
        lines.append(" ".join(map(str, s.ids)))
        lines.append(" ".join(map(str, s.pos)))
        if s.opt is not None:
            lines.append(" ".join(map(str, s.opt)))
        lines.append(" ".join(map(str, s.mask_pos)))
    open(path_m, "w").write("\n".join(lines) + "\n")


@pytest.mark.gpu
@pytest.mark.parametrize("prec", ["bf16", "fp32"])
def test_replay_forward_matches_engine(replay, prec):
    """New -> Forward -> Free from C on a small model: the logits are bit for
    bit those of the same library driven from Python (Engine.forward), and an
    input error comes back with forward.go's message."""
    from decide_amd import Engine
    from decide_amd.nn import Config, Sequence, build_sequence
    from decide_amd.synth import random_weights

    cfg = Config(hidden=256, intermediate=384, heads=4, layers=2, vocab=400, half_window=8,
                 layer_types=["full_attention", "sliding_attention"])
    w = random_weights(cfg, seed=21, std=0.05)
    rng = np.random.default_rng(3)
    batch = []
    for n, opts, indep in [(40, [3, 4, 5], True), (70, [6, 6], False)]:
        ids = [1] + list(rng.integers(3, 399, size=n)) + [2]
        for ln in opts:
            ids += [399] + list(rng.integers(3, 399, size=ln - 1))
        batch.append(build_sequence(np.array(ids + [2], np.int32), 399, independent=indep))
    p = 1 if prec == "bf16" else 0
    m, wb = replay.dir / f"m_{prec}.txt", replay.dir / f"w_{prec}.bin"
    write_manifest(m, wb, cfg, w, batch, p)
    print(f"case: replay forward {prec}", flush=True)
    out = replay(str(m), str(wb))
    assert out[1] == "ok 5", out[:3]
    got = np.array([struct.unpack("<f", bytes.fromhex(l.split()[1])[::-1])[0] for l in out[2:]], np.float32)
    with Engine(cfg, w, precision=prec) as eng:
        want = eng.forward(batch)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (got, want)
    bad = [batch[0], Sequence(ids=batch[1].ids, pos=batch[1].pos, opt=None, mask_pos=np.zeros(0, np.int32))]
    write_manifest(m, wb, cfg, w, bad, p)
    assert replay(str(m), str(wb))[1] == "error 2 nn: sequence 1 has no options"


def _logits(out):
    return np.array([struct.unpack("<f", bytes.fromhex(l.split()[1])[::-1])[0] for l in out if l.startswith("logit ")],
                    np.float32)


@pytest.mark.gpu
def test_replay_reference_fixture(replay, tiny_ref):
    """internal/gpunn/gpunn_test.go:119-164's check, through the binding's
    call sequence: the reference's own PyTorch fixture (tiny_ref.safetensors:
    its weights and its two packed sequences) through New -> Forward -> Free
    from C in the fp32 mode. The logits match the fixture's PyTorch logits at
    relErr <= 1e-4 (the reference test's bar) and the oracle's at
    1e-5 * (1 + |logit|)."""
    from conftest import rel_err, tiny_config, tiny_weights
    from decide_amd.nn import build_sequence

    tensors, meta = tiny_ref
    cfg = tiny_config(meta)
    w = tiny_weights(tensors, cfg)
    batch = [build_sequence(s["ids"], meta["mask_id"], s["independent"]) for s in meta["seqs"]]
    m, wb = replay.dir / "m_tiny.txt", replay.dir / "w_tiny.bin"
    write_manifest(m, wb, cfg, w, batch, 0)
    print("case: replay tiny_ref fixture fp32", flush=True)
    out = replay(str(m), str(wb))
    assert out[1] == f"ok {len(tensors['logits'])}", out[:3]
    got = _logits(out)
    err = rel_err(got, tensors["logits"])
    oracle_mod = __import__("oracle")
    oracle_mod.set_workers(4)
    want = oracle_mod.OracleModel(cfg, w).forward(batch)
    print(f"relErr against the PyTorch logits {err:.3g}; max |d| against the oracle "
          f"{float(np.max(np.abs(got.astype(np.float64) - want))):.3g}", flush=True)
    assert err <= 1e-4
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * (1 + np.abs(want)))


def _evaluate_manifest(path_m, path_w, cfg, w, precision, certify, qspecs, mask_id):
    write_manifest(path_m, path_w, cfg, w, [], precision)
    lines = open(path_m).read().splitlines()
    if certify:
        lines.insert(1, f"certify {certify!r}")
    for kind, nopt, ids, temp in qspecs:
        lines.append(f"question {kind} {nopt} {len(ids)} {temp!r}")
        lines.append(" ".join(map(str, ids)))
    lines.append(f"evaluate {mask_id} 1")
    open(path_m, "w").write("\n".join(lines) + "\n")


@pytest.mark.gpu
@pytest.mark.parametrize("prec,certify", [("fp32", 0.0), ("fp16", 1e-3)])
def test_replay_evaluate_matches_serial_oracle(replay, prec, certify):
    """The wired decide.Local's call from C: every question of one SystemOne
    call through ONE dn_evaluate (hipnn.Evaluate), in the fp32 validation
    mode and in the mode the wiring uses (fp16 + certified argmax, margin
    1e-3), against the serial oracle, which answers each question with its own
    Forward as local.go:126-204 does. Choice and Score argmaxes agree exactly;
    rounded probabilities within 1e-4 (fp32) / 2e-3 + 1e-4 (fp16)."""
    import oracle as orc

    from decide_amd import local as L
    from decide_amd.nn import config_from_dict
    from decide_amd.synth import random_weights
    from test_gpu_local import CAL, STATE, TINY, questions
    from test_local import MIN_MASK, byte_encode

    cfg = config_from_dict(TINY)
    w = random_weights(cfg, seed=7, std=0.05)
    cal = L.Calibration(CAL["temperature"], CAL["default"])
    state = L.format_state(STATE)
    qs = questions()
    specs = []
    for _, q in qs:
        kind, texts, ck = L._options(q)
        need = kind == L.DN_KIND_NOUL or len(texts) > 1
        ids = byte_encode(L.pack_text(state, q.instructions, texts)) if need else []
        specs.append((kind, len(texts), list(map(int, ids)), cal.temperature_for(ck)))
    m, wb = replay.dir / f"m_eval_{prec}.txt", replay.dir / f"w_eval_{prec}.bin"
    _evaluate_manifest(m, wb, cfg, w, {"fp32": 0, "fp16": 2}[prec], certify, specs, MIN_MASK)
    print(f"case: replay dn_evaluate {prec} certify {certify}", flush=True)
    out = replay(str(m), str(wb))
    assert out[1] == f"answers {len(qs)}", out[:3]
    orc.set_workers(4)
    om = orc.OracleModel(cfg, w)
    tol = 1e-4 + 1e-9 if prec == "fp32" else 2e-3 + 1e-4
    names = {L.DN_KIND_CHOICE: "choice", L.DN_KIND_SCORE: "score", L.DN_KIND_NOUL: "noul"}
    for (kind, nopt, ids, temp), line in zip(specs, out[2:]):
        f = line.split()
        assert f[0] == "answer"
        choice, conf, value = int(f[1]), float(f[2]), float(f[3])
        probs = np.array([float(x) for x in f[4:]])
        want = orc.evaluate_question(om, names[kind], nopt, ids, MIN_MASK, True, temp)
        assert len(probs) == len(want["probs"]) and choice == want["choice"], (line, want)
        if nopt:
            assert np.all(np.abs(probs - want["probs"]) <= tol), (line, want)
        assert abs(value - want["value"]) <= tol * max(1, nopt) ** 2, (line, want)
        assert abs(conf - want["confidence"]) <= 1e-3 + tol * max(1, nopt), (line, want)
