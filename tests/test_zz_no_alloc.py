"""aic_hip_grad_sqnorm_multi_noalloc, the allocation-free variant of aic_hip_grad_sqnorm_multi,
through the C-ABI: bit-identical results to the allocating entry on two calls in a row (the
second on a smaller input, with a non-finite value), no growth of the library's device pool,
and the size limit rejected on the host before anything is launched."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from autonomousaicore_amd import _lib  # noqa: E402
from tests.gpu_util import call, dev, host, ptr  # noqa: E402

MAX_BLOCKS = 1 << 17  # the fixed scratch of the no-alloc entry, in partial blocks


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _pool_bytes():
    a, p = C.c_int64(), C.c_int64()
    call("aic_hip_mem_stats", C.byref(a), C.byref(p))
    return a.value


def _sqnorm(entry, tensors, stream):
    ptrs = (C.c_void_p * len(tensors))(*[ptr(t) for t in tensors])
    sizes = (C.c_int64 * len(tensors))(*[t.numel() for t in tensors])
    sq = torch.full((1,), -1.0, dtype=torch.float64, device="cuda")
    nf = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    call(entry, ptrs, sizes, len(tensors), ptr(sq), ptr(nf), stream.cuda_stream)
    stream.synchronize()
    return float(host(sq)[0]), int(host(nf)[0])


def _blocks(n):
    return max(1, min((n + 4095) // 4096, 1024))


def test_noalloc_sqnorm_matches_allocating_entry():
    rng = np.random.default_rng(2024)
    # call 1: a 1024-block tensor, ragged sizes, a tensor not a multiple of 4, an empty one
    big = [rng.standard_normal(n).astype(np.float32) for n in (5_000_000, 1_000_003, 4099, 77, 0)]
    # call 2: smaller, with an infinity
    small = [rng.standard_normal(n).astype(np.float32) for n in (300_001, 5)]
    small[0][12345] = np.inf
    tb, ts = [dev(a) for a in big], [dev(a) for a in small]
    ref_b = float(sum((a.astype(np.float64) ** 2).sum() for a in big))

    s_noalloc, s_alloc = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for st in (s_noalloc, s_alloc):  # torch recycles streams: drop what the library cached for them
        call("aic_hip_mem_release_stream", st.cuda_stream)
    before = _pool_bytes()
    got_b = _sqnorm("aic_hip_grad_sqnorm_multi_noalloc", tb, s_noalloc)
    got_s = _sqnorm("aic_hip_grad_sqnorm_multi_noalloc", ts, s_noalloc)
    assert _pool_bytes() == before, "the no-alloc entry took memory from the library's pool"

    exp_b = _sqnorm("aic_hip_grad_sqnorm_multi", tb, s_alloc)
    assert _pool_bytes() > before  # control: the allocating entry takes its scratch on this stream
    exp_s = _sqnorm("aic_hip_grad_sqnorm_multi", ts, s_alloc)
    again = _sqnorm("aic_hip_grad_sqnorm_multi_noalloc", tb, s_noalloc)
    call("aic_hip_mem_release_stream", s_alloc.cuda_stream)
    assert _pool_bytes() == before  # the released scratch is back in the pool
    assert got_b == exp_b and got_s == exp_s  # bit for bit: the same partials in the same order
    assert got_b[1] == 0 and abs(got_b[0] - ref_b) < 1e-9 * ref_b
    assert got_s[1] == 1

    # and again on the first input after the smaller one: stale partials are never read
    assert again == exp_b


def test_noalloc_sqnorm_rejects_beyond_its_scratch():
    n = 4096 * 1024  # one full 1024-block tensor
    t = torch.ones(n, dtype=torch.float32, device="cuda")
    k = MAX_BLOCKS // 1024
    ptrs = (C.c_void_p * (k + 1))(*([ptr(t)] * (k + 1)))
    sizes = (C.c_int64 * (k + 1))(*([n] * (k + 1)))
    sq = torch.zeros(1, dtype=torch.float64, device="cuda")
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    # exactly at the limit: accepted
    call("aic_hip_grad_sqnorm_multi_noalloc", ptrs, sizes, k, ptr(sq), ptr(nf), s)
    assert float(host(sq)[0]) == float(k * n)
    # one tensor more: OutOfRange from the host check, nothing launched, outputs untouched
    sq.fill_(-2.0)
    with pytest.raises(_lib.AicError) as e:
        call("aic_hip_grad_sqnorm_multi_noalloc", ptrs, sizes, k + 1, ptr(sq), ptr(nf), s)
    assert e.value.code == 2 and "scratch" in str(e.value)
    assert float(host(sq)[0]) == -2.0
    assert sum(_blocks(n) for _ in range(k)) == MAX_BLOCKS
