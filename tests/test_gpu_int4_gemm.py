"""GPU tests of the GEMM with the INT4 weight operand dequantized inside the kernel (the QLoRA
base projections, QuantizedLinear::forward of src/nn/quantization.cpp:669-679 and its input
gradient), through the C-ABI.

aic_hip_int4_dequant_gemm reads the packed nibbles and group scales in the GEMM's operand load.
Its operand values are bf16(q * scale), the same values aic_hip_int4_dequantize writes (pinned
bit-exact against the oracle in test_gpu_qlora.py), and it runs the same MFMA tile schedule as
aic_hip_gemm, so on shapes where both choose the same tile (no split-K) the fused product must
equal dequantize-then-GEMM bit for bit.  The oracle checks the product itself at the bf16
rounding level, in both layouts, at the 1B projection shapes."""
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


def _qweight(orc, rng, rows, cols, G, f16):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    return orc.int4_quantize(w, G, scale_f16=f16)


def _fused(transW, M, N, K, alpha, x, pd, sd, f16, G, beta, c0, R, out_t):
    tdt = torch.float32 if out_t == F32 else torch.bfloat16
    cd = dev(c0, tdt) if c0 is not None else torch.empty((M, N), dtype=tdt, device="cuda")
    Rd = dev(R, tdt) if R is not None else None
    call("aic_hip_int4_dequant_gemm", transW, M, N, K, alpha, ptr(x), K, ptr(pd), ptr(sd), F16 if f16 else F32, G,
         beta, ptr(cd), N, ptr(Rd), N if R is not None else 0, BF16, out_t, stream())
    return host(cd)


def _staged(transW, M, N, K, alpha, x, pd, sd, f16, G, beta, c0, R, out_t):
    tdt = torch.float32 if out_t == F32 else torch.bfloat16
    w = torch.empty(N * K, dtype=torch.bfloat16, device="cuda")
    call("aic_hip_int4_dequantize", ptr(pd), ptr(sd), F16 if f16 else F32, N * K, G, ptr(w), BF16, stream())
    cd = dev(c0, tdt) if c0 is not None else torch.empty((M, N), dtype=tdt, device="cuda")
    Rd = dev(R, tdt) if R is not None else None
    call("aic_hip_gemm", 0, transW, M, N, K, alpha, ptr(x), K, ptr(w), K if transW else N, beta, ptr(cd), N, ptr(Rd),
         N if R is not None else 0, BF16, out_t, stream())
    return host(cd)


# (transW, M, N, K, G, f16 scales, out type, epilogue): the 1B q/k/v forward, down and gate/up
# input gradients (256x256 tiles), ragged M and N on 128x128 tiles and on 256x256 tiles (eight
# waves; with the epilogue, and fp32 output), fp32 outputs, alpha / beta / residual, groups of 64
# and 256; fp32 scales take the staged route (the kernel reads fp16 ones)
CASES = [
    (1, 8192, 6144, 2048, 128, True, BF16, False),
    (0, 8192, 5632, 2048, 128, True, BF16, False),
    (0, 8192, 2048, 11264, 128, True, BF16, False),
    (1, 8000, 4160, 1024, 128, True, BF16, True),
    (0, 4100, 8192, 1024, 64, True, F32, True),
    (1, 1000, 1000, 512, 64, True, F32, True),
    (0, 520, 384, 640, 256, True, F32, True),
    (1, 2048, 2048, 2048, 128, True, BF16, True),
    (0, 300, 128, 256, 64, True, BF16, True),
    (1, 256, 320, 384, 64, False, BF16, True),
]


@pytest.mark.parametrize("transW,M,N,K,G,f16,out_t,epi", CASES)
def test_int4_gemm_fused_equals_dequantize_then_gemm(orc, transW, M, N, K, G, f16, out_t, epi):
    print(f"int4 fused vs staged: transW {transW} M {M} N {N} K {K} G {G} f16 {f16} out {out_t} epi {epi}", flush=True)
    rng = np.random.default_rng(M + 3 * N + 7 * K + transW)
    rows, cols = (N, K) if transW else (K, N)
    packed, scales = _qweight(orc, rng, rows, cols, G, f16)
    x = dev(rng.standard_normal((M, K)).astype(np.float32), torch.bfloat16)
    pd, sd = dev(packed), dev(scales)
    alpha, beta = (0.75, 0.5) if epi else (1.0, 0.0)
    c0 = rng.standard_normal((M, N)).astype(np.float32) if epi else None
    R = rng.standard_normal((M, N)).astype(np.float32) if epi else None
    a = _fused(transW, M, N, K, alpha, x, pd, sd, f16, G, beta, c0, R, out_t)
    b = _staged(transW, M, N, K, alpha, x, pd, sd, f16, G, beta, c0, R, out_t)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"max |diff| {np.abs(a - b).max()}"


@pytest.mark.parametrize("transW,M,N,K", [(1, 512, 11264, 2048), (0, 512, 2048, 5632), (1, 256, 2048, 5632),
                                          (0, 256, 5632, 2048)])
def test_int4_gemm_matches_oracle_at_1b_projection_shapes(orc, transW, M, N, K):
    # gate/up forward, down-input-gradient-like, down forward and gate input gradient layouts
    print(f"int4 gemm vs oracle: transW {transW} M {M} N {N} K {K}", flush=True)
    rng = np.random.default_rng(11 + M + N + K + transW)
    rows, cols = (N, K) if transW else (K, N)
    packed, scales = _qweight(orc, rng, rows, cols, 128, True)
    W = orc.int4_dequantize(packed, scales, N * K, 128).reshape(rows, cols)
    x = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xd, pd, sd = dev(x, torch.bfloat16), dev(packed), dev(scales)
    y = _fused(transW, M, N, K, 1.0, xd, pd, sd, True, 128, 0.0, None, None, F32)
    Wb = bf16_round(W).astype(np.float64)
    ref = x.astype(np.float64) @ (Wb.T if transW else Wb)
    assert rel(y, ref) < 1e-5   # fp32 output of bf16 operands: accumulation order only


def test_int4_gemm_other_shapes_fall_back_to_staging(orc):
    # input gradient with N % 64 != 0 and a group of 32: the staged route, same result contract
    rng = np.random.default_rng(5)
    M, N, K, G = 96, 200, 128, 32
    packed, scales = _qweight(orc, rng, K, N, G, True)
    W = orc.int4_dequantize(packed, scales, N * K, G).reshape(K, N)
    x = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xd, pd, sd = dev(x, torch.bfloat16), dev(packed), dev(scales)
    y = _fused(0, M, N, K, 1.0, xd, pd, sd, True, G, 0.0, None, None, F32)
    ref = x.astype(np.float64) @ bf16_round(W).astype(np.float64)
    assert rel(y, ref) < 1e-5


# (T, d, K, r, seq, start, G): the q/k/v projection of 128-wide heads with the rank-r adapters of
# q, k and v side by side; 192 tiles of 256x256 take the INT4 kernel's rotary epilogue (with and
# without the adapters, and at a decode-style start position), 24 tiles the product and then
# the rope pass; quantization groups of 32 (not a multiple of 64: the operand-load
# dequantization cannot take them) dequantize the weight into scratch, then the product and rope
@pytest.mark.parametrize("T,d,K,r,seq,start,G", [(4096, 1024, 512, 16, 2048, 0, 128), (4096, 1024, 256, 0, 1024, 0, 128),
                                                 (4096, 1024, 256, 16, 4096, 3, 128), (1024, 512, 256, 16, 512, 0, 128),
                                                 (4096, 1024, 256, 16, 2048, 0, 32)])
def test_int4_gemm_rope_equals_product_then_rope(orc, T, d, K, r, seq, start, G):
    """aic_hip_int4_gemm_rope = the low-rank GEMM over the dequantized weight, then aic_hip_rope on
    the q and k columns: v columns bit-identical (the same products), q / k within one bf16
    rounding of the rotation of the same bf16 sum, and the oracle's RoPE of the float64 sum
    within the bf16 bound."""
    print(f"int4 gemm rope: T {T} d {d} K {K} r {r} seq {seq} start {start} G {G}", flush=True)
    rng = np.random.default_rng(T + d + K + r + start + G)
    hd, N = 128, 3 * d
    packed, scales = _qweight(orc, rng, N, K, G, True)
    W = bf16_round(orc.int4_dequantize(packed, scales, N * K, G).reshape(N, K))
    x = bf16_round(rng.standard_normal((T, K)).astype(np.float32))
    X2 = bf16_round(rng.standard_normal((T, 3 * max(r, 1))).astype(np.float32))
    Y2 = bf16_round((rng.standard_normal((N, max(r, 1))) / 4).astype(np.float32))
    cos_t = np.empty((start + seq, hd // 2), np.float32)
    sin_t = np.empty_like(cos_t)
    _lib.check(_lib.load().aic_hip_rope_tables(cos_t.ctypes.data, sin_t.ctypes.data, start + seq, hd, 10000.0))
    xd, pd, sd, Wd = dev(x, torch.bfloat16), dev(packed), dev(scales), dev(W, torch.bfloat16)
    X2d, Y2d, cd, snd = dev(X2, torch.bfloat16), dev(Y2, torch.bfloat16), dev(cos_t), dev(sin_t)
    ldx2 = X2.shape[1]
    fused = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_int4_gemm_rope", T, N, K, ptr(xd), K, ptr(pd), ptr(sd), G, ptr(X2d), ldx2, ptr(Y2d), Y2.shape[1], r,
         d, ptr(fused), N, 2 * d, hd, seq, start, ptr(cd), ptr(snd), stream())
    sep = torch.empty_like(fused)
    if r > 0:
        call("aic_hip_gemm_lowrank", 0, 1, T, N, K, 1.0, ptr(xd), K, ptr(Wd), K, ptr(X2d), ldx2, ptr(Y2d), Y2.shape[1],
             r, d, 0, 0.0, ptr(sep), N, None, 0, BF16, BF16, stream())
    else:
        call("aic_hip_gemm", 0, 1, T, N, K, 1.0, ptr(xd), K, ptr(Wd), K, 0.0, ptr(sep), N, None, 0, BF16, BF16,
             stream())
    call("aic_hip_rope", ptr(sep), N, T // seq, seq, 2 * d // hd, hd, start, ptr(cd), ptr(snd), 0, BF16, stream())
    f, g = host(fused), host(sep)
    np.testing.assert_array_equal(f[:, 2 * d:], g[:, 2 * d:])
    assert np.max(np.abs(f[:, :2 * d] - g[:, :2 * d]) / (np.abs(g[:, :2 * d]) + 1e-3)) < 1e-2
    assert rel(f[:, :2 * d], g[:, :2 * d]) < 2e-3
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    if r > 0:
        for s in range(3):
            ref[:, s * d:(s + 1) * d] += X2[:, s * r:(s + 1) * r].astype(np.float64) @ \
                Y2[s * d:(s + 1) * d].astype(np.float64).T
    qk = orc.rope_fwd(ref[:, :2 * d], T // seq, seq, 2 * d // hd, hd, start_pos=start)
    assert rel(f[:, :2 * d], qk) < 8e-3
    assert rel(f[:, 2 * d:], ref[:, 2 * d:]) < 8e-3
    again = torch.empty_like(fused)
    call("aic_hip_int4_gemm_rope", T, N, K, ptr(xd), K, ptr(pd), ptr(sd), G, ptr(X2d), ldx2, ptr(Y2d), Y2.shape[1], r,
         d, ptr(again), N, 2 * d, hd, seq, start, ptr(cd), ptr(snd), stream())
    np.testing.assert_array_equal(host(again), f)


# (T, f, K, r, G): the gate/up projection of the FFN with the gate and up adapters side by side
# (seg_n = f); 128 and 176 tiles of 256x256 take the INT4 kernel's SwiGLU epilogue, with and
# without the adapters
@pytest.mark.parametrize("T,f,K,r,G", [(4096, 1024, 512, 16, 128), (4096, 1024, 256, 0, 128),
                                       (2048, 2816, 512, 16, 64)])
def test_int4_gemm_swiglu_equals_product_then_swiglu(orc, T, f, K, r, G):
    """aic_hip_int4_gemm_swiglu: GU equal bit for bit to the low-rank GEMM over the dequantized
    weight (the same bf16 operand values, MFMA sequence and low-rank tail), H equal bit for bit to
    aic_hip_swiglu_fwd of that GU, and the float64 product within the bf16 bound."""
    print(f"int4 gemm swiglu: T {T} f {f} K {K} r {r} G {G}", flush=True)
    rng = np.random.default_rng(T + f + K + r + G)
    N = 2 * f
    packed, scales = _qweight(orc, rng, N, K, G, True)
    W = bf16_round(orc.int4_dequantize(packed, scales, N * K, G).reshape(N, K))
    x = bf16_round(rng.standard_normal((T, K)).astype(np.float32))
    X2 = bf16_round(rng.standard_normal((T, 2 * max(r, 1))).astype(np.float32))
    Y2 = bf16_round((rng.standard_normal((N, max(r, 1))) / 4).astype(np.float32))
    xd, pd, sd, Wd = dev(x, torch.bfloat16), dev(packed), dev(scales), dev(W, torch.bfloat16)
    X2d, Y2d = dev(X2, torch.bfloat16), dev(Y2, torch.bfloat16)
    ldx2 = X2.shape[1]
    gu = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")
    h = torch.empty((T, f), dtype=torch.bfloat16, device="cuda")
    call("aic_hip_int4_gemm_swiglu", T, f, K, ptr(xd), K, ptr(pd), ptr(sd), G, ptr(X2d), ldx2, ptr(Y2d), Y2.shape[1],
         r, f, ptr(gu), N, ptr(h), f, stream())
    sep = torch.empty_like(gu)
    if r > 0:
        call("aic_hip_gemm_lowrank", 0, 1, T, N, K, 1.0, ptr(xd), K, ptr(Wd), K, ptr(X2d), ldx2, ptr(Y2d), Y2.shape[1],
             r, f, 0, 0.0, ptr(sep), N, None, 0, BF16, BF16, stream())
    else:
        call("aic_hip_gemm", 0, 1, T, N, K, 1.0, ptr(xd), K, ptr(Wd), K, 0.0, ptr(sep), N, None, 0, BF16, BF16,
             stream())
    h2 = torch.empty_like(h)
    call("aic_hip_swiglu_fwd", ptr(sep), ptr(sep) + 2 * f, N, ptr(h2), f, T, f, BF16, stream())
    np.testing.assert_array_equal(host(gu), host(sep))
    np.testing.assert_array_equal(host(h), host(h2))
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    if r > 0:
        for s in range(2):
            ref[:, s * f:(s + 1) * f] += X2[:, s * r:(s + 1) * r].astype(np.float64) @ \
                Y2[s * f:(s + 1) * f].astype(np.float64).T
    assert rel(host(gu), ref) < 8e-3
    g, u = ref[:, :f], ref[:, f:]
    assert rel(host(h), g / (1.0 + np.exp(-g)) * u) < 2e-2
