"""GPU parity of the tensor primitives (strided copy, casts, broadcasting binary ops, unary
functions, reductions, cat, broadcast-gradient reduction) through the C-ABI, against the CPU
oracle (orc_*), which the CPU suite pins against the reference's tests/unit/test_ops.cpp,
test_tensor.cpp and test_shape.cpp known answers, numpy and torch.  Copies, casts, max / min
and + - * / are bit-exact; transcendental functions within a few ulp (the reference's own GPU
parity test allows 1e-4, tests/unit/test_ops.cpp:150-223); double-accumulated sums equal the
oracle's float result or differ by one ulp where double rounding in another order flips it."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from autonomousaicore_amd import _lib  # noqa: E402
from tests.gpu_util import call, dev, host, ptr, stream  # noqa: E402

F32, F16, BF16, I32, I64 = _lib.AIC_F32, _lib.AIC_F16, _lib.AIC_BF16, _lib.AIC_I32, _lib.AIC_I64


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _i64(v):
    a = np.ascontiguousarray(np.asarray(v, np.int64))
    return a, a.ctypes.data_as(C.POINTER(C.c_int64))


def _ulp_close(a, b, ulps=1):
    a = np.asarray(a, np.float32).ravel()
    b = np.asarray(b, np.float32).ravel()
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    return bool(np.all(np.abs(ia - ib) <= ulps) or np.allclose(a, b, rtol=0, atol=0))


@pytest.mark.parametrize("es,dtype", [(4, np.float32), (8, np.int64), (2, np.float16), (1, np.uint8)])
def test_strided_copy_views(orc, es, dtype):
    rng = np.random.default_rng(es)
    base = (rng.standard_normal(4000) * 100).astype(dtype)
    bd = dev(base)
    for off, shape, strides in [(0, [3, 2], [1, 3]), (7, [5, 4, 3], [1, 15, 5]), (3, [10, 20], [60, 2]),
                                (1, [2, 3, 4, 5], [1, 2, 6, 24]), (0, [37, 29], [29, 1]), (11, [4, 1, 6], [6, 99, 1])]:
        ref = orc.strided_copy(base, off, shape, strides)
        out = torch.empty(int(np.prod(shape)), dtype=bd.dtype, device="cuda")
        sh, shp = _i64(shape)
        st, stp = _i64(strides)
        call("aic_hip_strided_copy", ptr(bd), off, len(shape), shp, stp, es, ptr(out), stream())
        np.testing.assert_array_equal(host(out).reshape(shape), ref)


def _cast(x, frm, to, out_dtype):
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out = torch.empty(x.size, dtype=out_dtype, device="cuda")
    call("aic_hip_cast", ptr(xd), frm, ptr(out), to, x.size, stream())
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_casts_bit_exact(orc):
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
                        np.array([0.0, -0.0, 65504, 65519, 65520, 1e9, 2.0 ** -25, 2.0 ** -24 * 1.5, np.inf, -np.inf,
                                  np.nan], np.float32)]).astype(np.float32)
    x = np.concatenate([x, np.array([0x7F800001, 0xFFC12345, 0x7FBFFFFF], np.uint32).view(np.float32)])
    np.testing.assert_array_equal(_cast(x, F32, F16, torch.int16).view(np.uint16), orc.cast(x, "f16"))
    np.testing.assert_array_equal(_cast(x, F32, BF16, torch.int16).view(np.uint16), orc.cast(x, "bf16"))
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)              # every 16-bit pattern
    np.testing.assert_array_equal(_cast(h, F16, F32, torch.float32).view(np.uint32), orc.cast(h, "f32").view(np.uint32))
    np.testing.assert_array_equal(_cast(h, BF16, F32, torch.float32).view(np.uint32),
                                  orc.cast(h, "f32", bf16_from=True).view(np.uint32))
    xi = (rng.standard_normal(5000) * 1e5).astype(np.float32)
    np.testing.assert_array_equal(_cast(xi, F32, I64, torch.int64), orc.cast(xi, "i64"))
    np.testing.assert_array_equal(_cast(xi, F32, I32, torch.int32), orc.cast(xi, "i32"))
    iv = rng.integers(-2 ** 60, 2 ** 60, 5000)
    np.testing.assert_array_equal(_cast(iv, I64, F32, torch.float32), orc.cast(iv, "f32"))
    np.testing.assert_array_equal(_cast(iv, I64, I32, torch.int32), orc.cast(iv, "i32"))
    i32 = iv.astype(np.int32)
    np.testing.assert_array_equal(_cast(i32, I32, F32, torch.float32), orc.cast(i32, "f32"))
    np.testing.assert_array_equal(_cast(i32, I32, I64, torch.int64), orc.cast(i32, "i64"))
    lib = _lib.load()
    assert lib.aic_hip_cast(None, F16, None, BF16, 4, None) == 8 and b"not implemented" in lib.aic_hip_last_error()


BCAST = [((4, 1, 5), (3, 1)), ((2, 3, 4), (4,)), ((1,), (7, 6)), ((5, 1), (1, 6)), ((64, 33), (64, 33)),
         ((1000,), (1,)), ((8, 16, 128), (16, 1))]


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_binary_broadcast_bit_exact(orc, op):
    rng = np.random.default_rng(len(op))
    code = orc.BINARY[op]
    for sa, sb in BCAST:
        a = rng.standard_normal(sa).astype(np.float32)
        b = (rng.standard_normal(sb) + 3).astype(np.float32)
        ad, bd = dev(a), dev(b)
        ref = orc.binary(op, a, b)
        out = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
        s1, p1 = _i64(sa)
        t1, q1 = _i64([s // 4 for s in a.strides])
        s2, p2 = _i64(sb)
        t2, q2 = _i64([s // 4 for s in b.strides])
        call("aic_hip_binary", code, ptr(ad), 0, len(sa), p1, q1, ptr(bd), 0, len(sb), p2, q2, ptr(out), stream())
        np.testing.assert_array_equal(host(out), ref)
    # strided views with offsets: a transposed view of a base and a step-2 slice
    base = rng.standard_normal(100).astype(np.float32) + 2
    bd = dev(base)
    ref = orc.binary(op, base, base, (2, [3, 4], [1, 3]), (5, [4], [2]))
    out = torch.empty((3, 4), dtype=torch.float32, device="cuda")
    s1, p1 = _i64([3, 4])
    t1, q1 = _i64([1, 3])
    s2, p2 = _i64([4])
    t2, q2 = _i64([2])
    call("aic_hip_binary", code, ptr(bd), 2, 2, p1, q1, ptr(bd), 5, 1, p2, q2, ptr(out), stream())
    np.testing.assert_array_equal(host(out), ref)


def test_binary_rejects_incompatible_shapes():
    s1, p1 = _i64([2, 3, 4])
    s2, p2 = _i64([5, 4])
    lib = _lib.load()
    assert lib.aic_hip_binary(0, None, 0, 3, p1, p1, None, 0, 2, p2, p2, None, None) == 3


@pytest.mark.parametrize("op", ["neg", "abs", "exp", "log", "sqrt", "tanh", "sigmoid", "gelu", "silu"])
def test_unary(orc, op):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(100003) * 4).astype(np.float32)
    if op in ("log", "sqrt"):
        x = np.abs(x) + 1e-4
    ref = orc.unary(op, x)
    xd = dev(x)
    y = torch.empty_like(xd)
    call("aic_hip_unary", orc.UNARY[op], ptr(xd), ptr(y), x.size, stream())
    got = host(y)
    if op in ("neg", "abs", "sqrt"):
        np.testing.assert_array_equal(got, ref)
    else:
        np.testing.assert_allclose(got, ref, rtol=4e-6, atol=2e-7)
    # the reference's zero points (tests/unit/test_ops.cpp:71-91)
    if op in ("sigmoid", "tanh", "gelu", "silu", "exp"):
        z = dev(np.zeros(5, np.float32))
        y0 = torch.empty_like(z)
        call("aic_hip_unary", orc.UNARY[op], ptr(z), ptr(y0), 5, stream())
        assert np.all(host(y0) == {"sigmoid": 0.5, "tanh": 0.0, "gelu": 0.0, "silu": 0.0, "exp": 1.0}[op])


@pytest.mark.parametrize("n", [1, 5, 1000, 1 << 20, 3_000_001])
def test_reduce_all(orc, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) + 0.3).astype(np.float32)
    xd = dev(x)
    out = torch.empty(1, dtype=torch.float32, device="cuda")
    for op in ("sum", "mean", "max", "min"):
        call("aic_hip_reduce_all", orc.REDUCE[op], ptr(xd), n, ptr(out), stream())
        got, ref = host(out)[0], orc.reduce_all(op, x)
        if op in ("max", "min"):
            assert got == ref
        else:
            assert _ulp_close(got, ref), (op, got, ref)


@pytest.mark.parametrize("shape", [(2, 3), (6, 50, 7), (4, 1000), (3, 8, 1, 257), (2049,), (5, 4, 3, 2)])
def test_reduce_dim(orc, shape):
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    x.ravel()[::97] = np.nan if len(shape) > 2 else x.ravel()[::97]   # NaN never wins max / min
    xd = dev(x)
    sh, shp = _i64(shape)
    for d in range(-1, len(shape)):
        for op in ("sum", "mean", "max", "min"):
            ref = orc.reduce_dim(op, x, d)
            out = torch.empty(max(ref.size, 1), dtype=torch.float32, device="cuda")
            call("aic_hip_reduce_dim", orc.REDUCE[op], ptr(xd), len(shape), shp, d, ptr(out), stream())
            got = host(out)[:ref.size].reshape(ref.shape)
            if op in ("max", "min"):
                np.testing.assert_array_equal(got, ref)
            else:
                assert _ulp_close(got[np.isfinite(ref)], ref[np.isfinite(ref)]), (op, d)
                np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))


def test_cat(orc):
    rng = np.random.default_rng(5)
    for d, shapes in [(1, [(2, 1, 3), (2, 4, 3), (2, 2, 3)]), (0, [(3, 5), (1, 5), (4, 5)]), (-1, [(4, 2), (4, 7)])]:
        parts = [rng.standard_normal(s).astype(np.float32) for s in shapes]
        ref = orc.cat(parts, d)
        dd = d + len(shapes[0]) if d < 0 else d
        outer = int(np.prod(shapes[0][:dd]))
        inner = int(np.prod(shapes[0][dd + 1:]))
        pd = [dev(p) for p in parts]
        srcs = (C.c_void_p * len(pd))(*[ptr(t) for t in pd])
        mids, mp = _i64([s[dd] for s in shapes])
        out = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
        call("aic_hip_cat", srcs, mp, len(pd), outer, inner, 4, ptr(out), stream())
        np.testing.assert_array_equal(host(out), ref)


def test_sum_to_shape(orc):
    rng = np.random.default_rng(6)
    g = rng.standard_normal((4, 2, 3, 5)).astype(np.float32)
    gd = dev(g)
    sh, shp = _i64(g.shape)
    for target in [(3, 5), (1, 5), (3, 1), (2, 1, 5), (1, 1), (), (4, 2, 3, 5), (1, 2, 1, 1)]:
        ref = orc.sum_to_shape(g, target)
        tg, tgp = _i64(list(target) if target else [0])
        out = torch.empty(max(ref.size, 1), dtype=torch.float32, device="cuda")
        call("aic_hip_sum_to_shape", ptr(gd), g.ndim, shp, len(target), tgp, ptr(out), stream())
        got = host(out)[:ref.size].reshape(ref.shape)
        assert _ulp_close(got, ref), target
