"""GPU parity of the QLoRA path (INT4-symmetric quantize / dequantize, the dequantizing GEMM, the
LoRA adapter forward / backward and merge) through the C-ABI, against the CPU oracle
(orc_int4_*, orc_lora_*), which the CPU suite pins against the reference's known answers
(tests/unit/test_quantization.cpp, tests/unit/test_lora.cpp), closed forms and float64 autograd.
Packed bytes, scales and dequantized values must be bit-exact; fp32 products at the reference
tolerances; bf16 at the bf16 rounding level."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from autonomousaicore_amd import _lib  # noqa: E402
from tests.gpu_util import bf16_round, call, dev, host, ptr, rel, stream  # noqa: E402

F32, F16, BF16 = _lib.AIC_F32, _lib.AIC_F16, _lib.AIC_BF16


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _n_groups(n, G):
    g = n if (G <= 0 or G > n) else G
    return (n + g - 1) // g


def _quantize(x, G, f16):
    n = x.size
    xd = dev(x.ravel())
    packed = torch.full(((n + 1) // 2,), 0xAB, dtype=torch.uint8, device="cuda")
    scales = torch.empty(_n_groups(n, G), dtype=torch.float16 if f16 else torch.float32, device="cuda")
    call("aic_hip_int4_quantize", ptr(xd), n, G, ptr(packed), ptr(scales), F16 if f16 else F32, stream())
    return packed, scales


def _dequant(packed, scales, n, G, out_t):
    out = torch.empty(n, dtype=torch.float32 if out_t == F32 else torch.bfloat16, device="cuda")
    call("aic_hip_int4_dequantize", ptr(packed), ptr(scales), F16 if scales.dtype == torch.float16 else F32, n, G,
         ptr(out), out_t, stream())
    return out


# the 1B gate/up projection at full size, the test_quantization.cpp case, odd and partial groups,
# one group over the tensor, a single element
QCASES = [((5632, 2048), 128), ((64, 128), 32), ((1001,), 64), ((777,), 6), ((513,), 0), ((1,), 128), ((3, 50), 10)]


@pytest.mark.parametrize("shape,G", QCASES)
@pytest.mark.parametrize("f16", [False, True])
def test_int4_quantize_dequantize_bit_exact(orc, shape, G, f16):
    rng = np.random.default_rng(int(np.prod(shape)) + G + f16)
    x = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    x.ravel()[: min(x.size, 300)] *= 1e-6                       # tiny groups: floor and fp16-subnormal scales
    if x.size >= 8:
        x.ravel()[5] = 2.5 * np.abs(x.ravel()[:G or x.size]).max() / 7  # near a half step
    packed, scales = _quantize(x, G, f16)
    r_packed, r_scales = orc.int4_quantize(x, G, scale_f16=f16)
    np.testing.assert_array_equal(host(packed), r_packed)
    np.testing.assert_array_equal(host(scales).view(np.uint16 if f16 else np.uint32),
                                  r_scales.view(np.uint16 if f16 else np.uint32))
    ref = orc.int4_dequantize(r_packed, r_scales, x.size, G)
    np.testing.assert_array_equal(host(_dequant(packed, scales, x.size, G, F32)), ref)
    np.testing.assert_array_equal(host(_dequant(packed, scales, x.size, G, BF16)), bf16_round(ref))


def test_int4_dequant_every_byte(orc):
    # all 256 bytes under every scale position of a G = 8 layout (vector path) and G = 6 (scalar path)
    packed = np.tile(np.arange(256, dtype=np.uint8), 4)
    n = 2 * packed.size
    for G in (8, 6):
        scales = np.linspace(0.5, 3.0, _n_groups(n, G)).astype(np.float32)
        got = host(_dequant(dev(packed), dev(scales), n, G, F32))
        np.testing.assert_array_equal(got, orc.int4_dequantize(packed, scales, n, G))


@pytest.mark.parametrize("is_signed", [True, False])
@pytest.mark.parametrize("n,G,zp_kind", [(2047, 3, "int"), (4096, 0, "frac"), (1 << 20, 128, "int"),
                                         (1001, 2000, "none"), (777, 7, "frac"), (1, 128, "int")])
def test_int4_dequantize_zp_matches_oracle(orc, is_signed, n, G, zp_kind):
    """aic_hip_int4_dequantize_zp (launch_dequantize_int4 with zero points or unsigned nibbles):
    bit-exact against the oracle, odd and <= 0 group sizes, fractional zero points."""
    print(f"int4 dequantize zp: n {n} G {G} zp {zp_kind} signed {is_signed}", flush=True)
    rng = np.random.default_rng(n + G + is_signed)
    packed = rng.integers(0, 256, (n + 1) // 2).astype(np.uint8)
    ng = (n + G - 1) // G if G > 0 else 1
    scales = rng.uniform(1e-3, 2.0, ng).astype(np.float32)
    zp = {"none": None, "int": rng.integers(0, 16, ng).astype(np.float32),
          "frac": rng.uniform(-2.0, 17.0, ng).astype(np.float32)}[zp_kind]
    out = torch.full((n,), 7.0, dtype=torch.float32, device="cuda")
    pd, sd, zd = dev(packed), dev(scales), (dev(zp) if zp is not None else None)  # alive through the call
    call("aic_hip_int4_dequantize_zp", ptr(pd), ptr(sd), ptr(zd), 1 if is_signed else 0, n, G, ptr(out), stream())
    np.testing.assert_array_equal(host(out), orc.int4_dequantize_zp(packed, scales, zp, is_signed, n, G))


def _qweight(orc, rng, out, inn, G, f16, std=0.02):
    """An INT4 weight [out, in] quantized by the oracle: packed bytes and scales."""
    w = (rng.standard_normal((out, inn)) * std).astype(np.float32)
    return orc.int4_quantize(w, G, scale_f16=f16)


@pytest.mark.parametrize("transW", [1, 0])
@pytest.mark.parametrize("M,N,K", [(256, 384, 512), (100, 72, 136)])
def test_int4_dequant_gemm_fp32(orc, transW, M, N, K):
    rng = np.random.default_rng(M + N + K + transW)
    wshape = (N, K) if transW else (K, N)
    G = 128 if (N * K) % 128 == 0 else 8
    packed, scales = _qweight(orc, rng, *wshape, G, True)
    W = orc.int4_dequantize(packed, scales, N * K, G).reshape(wshape)
    x = rng.standard_normal((M, K)).astype(np.float32)
    R = rng.standard_normal((M, N)).astype(np.float32)
    c0 = rng.standard_normal((M, N)).astype(np.float32)
    xd, Rd, cd, pd, sd = dev(x), dev(R), dev(c0), dev(packed), dev(scales)   # kept alive across the call
    call("aic_hip_int4_dequant_gemm", transW, M, N, K, 0.5, ptr(xd), K, ptr(pd), ptr(sd), F16, G, 0.25, ptr(cd), N,
         ptr(Rd), N, F32, F32, stream())
    ref = 0.5 * (x.astype(np.float64) @ (W.T if transW else W).astype(np.float64)) + 0.25 * c0 + R
    assert rel(host(cd), ref) < 1e-5


def test_int4_dequant_gemm_bf16_1b_shape(orc):
    # the 1B q/k/v projection: y = x deq(W)^T, x [2048, 2048] bf16, W INT4 G=128 fp16 scales
    rng = np.random.default_rng(7)
    M, N, K = 2048, 2048, 2048
    packed, scales = _qweight(orc, rng, N, K, 128, True)
    W = orc.int4_dequantize(packed, scales, N * K, 128).reshape(N, K)
    x = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    xd, pd, sd = dev(x, torch.bfloat16), dev(packed), dev(scales)
    call("aic_hip_int4_dequant_gemm", 1, M, N, K, 1.0, ptr(xd), K, ptr(pd), ptr(sd), F16, 128, 0.0, ptr(y), N, None, 0,
         BF16, BF16, stream())
    ref = x.astype(np.float64) @ bf16_round(W).astype(np.float64).T
    assert rel(host(y), ref) < 4e-3


class _QLoRA:
    def __init__(self, inn, out, r, alpha, G, dtype):
        self.h = C.c_void_p()
        call("aic_qlora_linear_create", inn, out, r, alpha, G, F16, dtype, C.byref(self.h))

    def __enter__(self):
        return self

    def __exit__(self, *a):
        call("aic_qlora_linear_destroy", self.h)


def _qlora_run(x, packed, scales, A, Bm, alpha, G, dy, dtype, R=None, acc_init=None):
    T, inn = x.shape
    out, r = Bm.shape
    tdt = torch.float32 if dtype == F32 else torch.bfloat16
    with _QLoRA(inn, out, r, alpha, G, dtype) as m:
        xd, Ad, Bd = dev(x, tdt), dev(A, tdt), dev(Bm, tdt)
        pd, sd = dev(packed), dev(scales)
        Rd = dev(R, tdt) if R is not None else None
        y = torch.empty((T, out), dtype=tdt, device="cuda")
        call("aic_qlora_linear_forward", m.h, ptr(xd), T, ptr(pd), ptr(sd), ptr(Ad), ptr(Bd), ptr(Rd), ptr(y), stream())
        dyd = dev(dy, tdt)
        dx = torch.empty((T, inn), dtype=tdt, device="cuda")
        dA = dev(acc_init[0]) if acc_init else torch.full((r, inn), 7.0, device="cuda")
        dB = dev(acc_init[1]) if acc_init else torch.full((out, r), 7.0, device="cuda")
        call("aic_qlora_linear_backward", m.h, ptr(dyd), ptr(dx), ptr(dA), ptr(dB), 1 if acc_init else 0, stream())
        return host(y), host(dx), host(dA), host(dB)


@pytest.mark.parametrize("T,inn,out,r", [(128, 256, 192, 16), (96, 128, 320, 8), (64, 64, 64, 1)])
def test_qlora_linear_fp32_matches_oracle(orc, T, inn, out, r):
    rng = np.random.default_rng(T + inn + out + r)
    G, alpha = 64, 32.0
    packed, scales = _qweight(orc, rng, out, inn, G, True, std=0.05)
    W = orc.int4_dequantize(packed, scales, out * inn, G).reshape(out, inn)
    x = rng.standard_normal((T, inn)).astype(np.float32)
    A = rng.uniform(-1 / np.sqrt(inn), 1 / np.sqrt(inn), (r, inn)).astype(np.float32)
    Bm = (0.1 * rng.standard_normal((out, r))).astype(np.float32)
    dy = rng.standard_normal((T, out)).astype(np.float32)
    R = rng.standard_normal((T, out)).astype(np.float32)
    y, dx, dA, dB = _qlora_run(x, packed, scales, A, Bm, alpha, G, dy, F32, R=R)
    y_ref, _ = orc.lora_fwd(x, W, A, Bm, alpha / r, 1, T)
    r_dx, r_dA, r_dB = orc.lora_bwd(x, W, A, Bm, alpha / r, dy, 1, T)
    assert rel(y, y_ref + R) < 1e-5
    assert rel(dx, r_dx) < 1e-4
    assert rel(dA, r_dA) < 1e-4
    assert rel(dB, r_dB) < 1e-4
    # accumulate adds to existing adapter gradients (AccumulateGrad)
    init = (rng.standard_normal(A.shape).astype(np.float32), rng.standard_normal(Bm.shape).astype(np.float32))
    _, _, dA2, dB2 = _qlora_run(x, packed, scales, A, Bm, alpha, G, dy, F32, acc_init=init)
    assert rel(dA2, r_dA + init[0]) < 1e-4 and rel(dB2, r_dB + init[1]) < 1e-4


def test_qlora_zero_b_equals_the_quantized_base(orc):
    # tests/unit/test_lora.cpp:58-73: with B = 0 the output is the base projection, bit for bit
    rng = np.random.default_rng(3)
    T, inn, out, r, G = 128, 256, 128, 16, 128
    packed, scales = _qweight(orc, rng, out, inn, G, True)
    x = rng.standard_normal((T, inn)).astype(np.float32)
    A = rng.uniform(-0.06, 0.06, (r, inn)).astype(np.float32)
    y, *_ = _qlora_run(x, packed, scales, A, np.zeros((out, r), np.float32), 32.0, G,
                       np.zeros((T, out), np.float32), F32)
    base = torch.empty((T, out), dtype=torch.float32, device="cuda")
    xd, pd, sd = dev(x), dev(packed), dev(scales)
    call("aic_hip_int4_dequant_gemm", 1, T, out, inn, 1.0, ptr(xd), inn, ptr(pd), ptr(sd), F16, G, 0.0, ptr(base), out,
         None, 0, F32, F32, stream())
    np.testing.assert_array_equal(y, host(base))


def test_lora_merge_matches_unmerged(orc):
    # tests/unit/test_lora.cpp:107-143: merged forward == unmerged forward (1e-4); unmerge restores W
    rng = np.random.default_rng(4)
    T, inn, out, r, G, alpha = 16, 32, 48, 4, 32, 8.0
    packed, scales = _qweight(orc, rng, out, inn, G, True, std=0.2)
    W = orc.int4_dequantize(packed, scales, out * inn, G).reshape(out, inn)
    x = rng.standard_normal((T, inn)).astype(np.float32)
    A = rng.uniform(-0.2, 0.2, (r, inn)).astype(np.float32)
    Bm = rng.uniform(-0.5, 0.5, (out, r)).astype(np.float32)
    y, *_ = _qlora_run(x, packed, scales, A, Bm, alpha, G, np.zeros((T, out), np.float32), F32)
    Wd, Ad, Bd = dev(W), dev(A), dev(Bm)
    call("aic_hip_lora_merge", ptr(Wd), ptr(Ad), ptr(Bd), inn, out, r, alpha / r, 1, F32, stream())
    np.testing.assert_allclose(host(Wd), orc.lora_merge(W, A, Bm, alpha / r), rtol=0, atol=2e-6)
    ym = torch.empty((T, out), dtype=torch.float32, device="cuda")
    xd = dev(x)
    call("aic_hip_gemm", 0, 1, T, out, inn, 1.0, ptr(xd), inn, ptr(Wd), inn, 0.0, ptr(ym), out, None, 0, F32, F32,
         stream())
    assert np.max(np.abs(host(ym) - y)) < 1e-4
    call("aic_hip_lora_merge", ptr(Wd), ptr(Ad), ptr(Bd), inn, out, r, alpha / r, -1, F32, stream())
    assert np.max(np.abs(host(Wd) - W)) < 1e-6


def test_qlora_linear_bf16_close_to_fp32_oracle(orc):
    # the QLoRA configuration's projection widths scaled down: rank 16, alpha 32, G 128, fp16 scales
    rng = np.random.default_rng(5)
    T, inn, out, r, G, alpha = 512, 512, 1408, 16, 128, 32.0
    packed, scales = _qweight(orc, rng, out, inn, G, True)
    W = orc.int4_dequantize(packed, scales, out * inn, G).reshape(out, inn)
    x, A, Bm, dy = (bf16_round(a) for a in (rng.standard_normal((T, inn)).astype(np.float32),
                                           rng.uniform(-1 / np.sqrt(inn), 1 / np.sqrt(inn), (r, inn)).astype(np.float32),
                                           (0.02 * rng.standard_normal((out, r))).astype(np.float32),
                                           rng.standard_normal((T, out)).astype(np.float32)))
    y, dx, dA, dB = _qlora_run(x, packed, scales, A, Bm, alpha, G, dy, BF16)
    y_ref, _ = orc.lora_fwd(x, bf16_round(W), A, Bm, alpha / r, 1, T)
    r_dx, r_dA, r_dB = orc.lora_bwd(x, bf16_round(W), A, Bm, alpha / r, dy, 1, T)
    assert rel(y, y_ref) < 1e-2
    assert rel(dx, r_dx) < 1e-2
    assert rel(dA, r_dA) < 2e-2
    assert rel(dB, r_dB) < 2e-2
