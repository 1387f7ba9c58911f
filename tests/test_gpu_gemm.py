"""GEMM parity on the GPU: dn_gemm_f32 (blas.Sgemm semantics, fp32 MFMA)
against the oracle's Go-order sgemm, and the bf16 device GEMM against a
float64 product of the same bf16 operands."""
import math

import numpy as np
import pytest

import oracle
from test_oracle import SHAPES, naive

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    from decide_amd import Engine, NoGPUError
    from decide_amd.nn import Config

    cfg = Config(hidden=256, intermediate=384, heads=4, layers=1, vocab=8, layer_types=["full_attention"])
    try:
        e = Engine(cfg, None, precision="fp32")
    except NoGPUError:
        pytest.skip("no GPU")
    yield e
    e.close()


def abs_bound(ta, tb, M, N, K, A, lda, B, ldb):
    """sum_k |a_ik * b_kj|: the scale of the rounding error of any fp32 summation order."""
    return naive(ta, tb, M, N, K, np.abs(A), lda, np.abs(B), ldb)


@pytest.mark.parametrize("shape", SHAPES)
def test_gemm_f32_matches_oracle(eng, shape):
    """TestSgemm / TestGemmMatchesCPU shapes, all transposes x accumulate.
    Bar: |gpu - oracle| <= 1e-5 * sum_k |a b| (+ |C0| * 2^-23 when accumulating)."""
    rng = np.random.default_rng(11)
    M, N, K = shape
    for ta in (False, True):
        for tb in (False, True):
            lda = M if ta else K
            ldb = K if tb else N
            A = rng.standard_normal(M * K, dtype=np.float32)
            B = rng.standard_normal(K * N, dtype=np.float32)
            bound = abs_bound(ta, tb, M, N, K, A, lda, B, ldb).reshape(-1)
            for acc in (False, True):
                C0 = rng.standard_normal(M * N, dtype=np.float32)
                want = C0.copy()
                oracle.sgemm(ta, tb, M, N, K, A, lda, B, ldb, want, N, acc, workers=8)
                got = C0.copy()
                eng.gemm_f32(ta, tb, M, N, K, A, lda, B, ldb, got, N, acc)
                tol = 1e-5 * bound + (np.abs(C0) * 2.0 ** -23 if acc else 0) + 1e-30
                err = np.abs(got.astype(np.float64) - want)
                assert np.all(err <= tol), (shape, ta, tb, acc, float(np.max(err / tol)))
                # and the reference test's own bar against exact float64
                exact = naive(ta, tb, M, N, K, A, lda, B, ldb).reshape(-1) + (C0 if acc else 0)
                assert np.max(np.abs(got - exact)) <= 1e-3 * math.sqrt(K + 1)


def test_gemm_f32_leading_dims_untouched(eng):
    """TestSgemmLeadingDims / cuda gemm_test.go:78-83: padding columns untouched."""
    rng = np.random.default_rng(4)
    M, N, K = 20, 30, 40
    lda, ldb, ldc = K + 3, N + 5, N + 7
    A = rng.standard_normal(M * lda, dtype=np.float32)
    B = rng.standard_normal(K * ldb, dtype=np.float32)
    C = np.full(M * ldc, 7.0, np.float32)
    eng.gemm_f32(False, False, M, N, K, A, lda, B, ldb, C, ldc, False)
    C2 = C.reshape(M, ldc)
    assert np.max(np.abs(C2[:, :N] - naive(False, False, M, N, K, A, lda, B, ldb))) <= 1e-3
    assert np.all(C2[:, N:] == 7.0)


def test_gemm_cfg1(eng):
    """cfg1: fp32 X[512x768] . W^T, W[2304x768]; X ~ N(0,1), W ~ N(0,0.02), seed 0,
    against the Go-order AVX2 sgemm. Bar: rtol 1e-5 on the error-bound scale,
    |d_ij| <= 1e-5 * sum_k |x_ik w_jk| (plain elementwise rtol is ill-posed
    where the dot product cancels), and elementwise rtol 1e-5 on the entries
    that are not cancellation-dominated (|ref| >= 0.1 * sum_k |x w|)."""
    rng = np.random.default_rng(0)
    M, N, K = 512, 2304, 768
    X = rng.standard_normal(M * K, dtype=np.float32)
    W = (rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    want = np.zeros(M * N, np.float32)
    oracle.sgemm(False, True, M, N, K, X, K, W, K, want, N, False, workers=8)
    got = np.zeros(M * N, np.float32)
    eng.gemm_f32(False, True, M, N, K, X, K, W, K, got, N, False)
    bound = (np.abs(X.reshape(M, K)).astype(np.float64) @ np.abs(W.reshape(N, K)).T.astype(np.float64)).reshape(-1)
    err = np.abs(got.astype(np.float64) - want)
    ratio = float(np.max(err / (1e-5 * bound)))
    wellcond = np.abs(want) >= 0.1 * bound
    rel = float(np.max(err[wellcond] / np.abs(want[wellcond])))
    big = np.abs(want) > 1e-3 * np.abs(want).max()
    rel_all = float(np.max(err[big] / np.abs(want[big])))
    print(f"cfg1: max err/(1e-5*sum|xw|) = {ratio:.3f}, max rel (well-conditioned, {int(wellcond.sum())} entries) "
          f"= {rel:.3g}, max rel (|ref| > 1e-3 max) = {rel_all:.3g}")
    assert ratio <= 1.0 and rel <= 1e-5


@pytest.mark.parametrize("prec", ["bf16", "fp16"])
@pytest.mark.parametrize("M,N,K", [(64, 2304, 768), (112, 2304, 768), (1000, 2304, 768), (2048, 2304, 768),
                                   (3000, 768, 2304), (5000, 768, 1152), (9000, 768, 768)])
def test_gemm_16bit_device(eng, prec, M, N, K):
    """bf16 / fp16 operands, fp32 accumulate: against float64 of the same
    16-bit values. Shapes cover every tile config of the fp32 epilogue:
    whole-K small-M, 64 x 128, 64 x 192 and the large-M tiles of the
    768-wide residual GEMMs (ragged last row tiles)."""
    import torch

    dt = torch.bfloat16 if prec == "bf16" else torch.float16
    g = torch.Generator().manual_seed(M)
    A = torch.randn(M, K, generator=g).to(dt)
    B = (torch.randn(N, K, generator=g) * 0.02).to(dt)
    exact = A.double() @ B.double().T
    bound = A.double().abs() @ B.double().abs().T
    dA, dB = A.cuda(), B.cuda()
    dC = torch.zeros(M, N, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    eng.gemm_device(prec, M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr())
    eng.synchronize()
    err = (dC.cpu().double() - exact).abs()
    assert float((err / (1e-5 * bound + 1e-30)).max()) <= 1.0


@pytest.mark.parametrize("prec", ["bf16", "fp16"])
@pytest.mark.parametrize("M,N,K", [(100, 2304, 768), (3000, 2304, 768), (20000, 2304, 768), (12000, 1536, 768)])
def test_gemm_16bit_device_store(eng, prec, M, N, K):
    """dn_gemm_device_store (the QKV epilogue: output rounded to the operand
    type) at every tile config of that epilogue: small M, medium, the
    large-M 256 x 128 tiles and N = 1536 (the last layer's K and V). Each
    output must be the 16-bit rounding of a value within the fp32 error
    bound of the float64 product, i.e. within half an output ulp plus that
    bound; and it must equal the fp32-output GEMM (dn_gemm_device) rounded to
    the same type, bit for bit (the same MFMA sums, rounded once)."""
    import torch

    dt = torch.bfloat16 if prec == "bf16" else torch.float16
    g = torch.Generator().manual_seed(M + N)
    A = torch.randn(M, K, generator=g).to(dt)
    B = (torch.randn(N, K, generator=g) * 0.02).to(dt)
    dA, dB = A.cuda(), B.cuda()
    dC = torch.zeros(M, N, dtype=dt, device="cuda")
    dF = torch.zeros(M, N, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    eng.gemm_device_store(prec, M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr())
    eng.gemm_device(prec, M, N, K, dA.data_ptr(), dB.data_ptr(), dF.data_ptr())
    eng.synchronize()
    assert torch.equal(dC.cpu(), dF.cpu().to(dt))
    exact = A.double() @ B.double().T
    bound = A.double().abs() @ B.double().abs().T
    # half an ulp: 2^-8 (bf16, 8-bit significand) or 2^-11 (fp16) relative,
    # 2^-25 absolute below fp16's normal range
    half_ulp = exact.abs() * (2.0 ** -8 if prec == "bf16" else 2.0 ** -11) + 2.0 ** -25
    err = (dC.cpu().double() - exact).abs()
    assert float((err / (1e-5 * bound + half_ulp * 1.0001)).max()) <= 1.0


@pytest.mark.parametrize("prec", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("M,N,K", [(1, 2304, 768), (31, 768, 1152), (33, 384, 768), (64, 2304, 768),
                                   (65, 768, 768), (112, 768, 1152), (128, 2304, 64), (100, 128, 4096)])
def test_gemm_small_m(eng, prec, M, N, K):
    """M <= 128 runs the small-M kernel (each workgroup owns all of K; its
    waves' partial tiles are summed through LDS in a fixed order). Same bar as
    above, C += accumulate checked, and two calls in a row must agree bit for
    bit (the reduction order does not depend on timing)."""
    import torch

    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[prec]
    g = torch.Generator().manual_seed(M * 7 + N + K)
    A = torch.randn(M, K, generator=g).to(dt)
    B = (torch.randn(N, K, generator=g) * 0.02).to(dt)
    C0 = torch.randn(M, N, generator=g)
    exact = A.double() @ B.double().T + C0.double()
    bound = A.double().abs() @ B.double().abs().T + C0.double().abs() * 2.0 ** -23
    dA, dB = A.cuda(), B.cuda()
    outs = []
    for _ in range(2):
        dC = C0.clone().cuda()
        torch.cuda.synchronize()
        eng.gemm_device(prec, M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), accumulate=True)
        eng.synchronize()
        outs.append(dC.cpu())
    err = (outs[0].double() - exact).abs()
    assert float((err / (1e-5 * bound + 1e-30)).max()) <= 1.0
    assert torch.equal(outs[0], outs[1])


def test_mfma_calibrate(eng):
    """dn_mfma_calibrate returns a plausible rate for both operand modes (the
    register-only loop of the bench's attainable-peak line), in bf16 and fp16
    (below the 2.5 PFLOP/s peak) and fp32 (below 157.3 TFLOP/s); other modes
    are refused."""
    from decide_amd import InvalidArgument

    changing, constant = eng.mfma_calibrate(0), eng.mfma_calibrate(1)
    print(f"attainable bf16 MFMA: changing operands {changing:.0f}, constant {constant:.0f} TFLOP/s")
    assert 100.0 < changing < 2600.0 and 100.0 < constant < 2600.0
    c32, k32 = eng.mfma_calibrate(2), eng.mfma_calibrate(3)
    print(f"attainable fp32 MFMA: changing operands {c32:.1f}, constant {k32:.1f} TFLOP/s")
    assert 10.0 < c32 < 160.0 and 10.0 < k32 < 160.0
    c16, k16 = eng.mfma_calibrate(4), eng.mfma_calibrate(5)
    print(f"attainable fp16 MFMA: changing operands {c16:.0f}, constant {k16:.0f} TFLOP/s")
    assert 100.0 < c16 < 2600.0 and 100.0 < k16 < 2600.0
    with pytest.raises(InvalidArgument):
        eng.mfma_calibrate(6)
