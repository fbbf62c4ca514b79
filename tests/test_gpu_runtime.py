"""The runtime entries of the C-ABI on the GPU: the stream-ordered allocator
(aic_hip_mem_alloc_async / free_async / stats, replacing DeviceMemoryPool::allocate_on_stream
and deallocate_on_stream, include/memory/memory_pool.hpp:120-155) and the synchronous copy
(aic_hip_memcpy_sync, the reference's raw cudaMemcpy calls)."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from autonomousaicore_amd import _lib  # noqa: E402
from tests.gpu_util import call  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


def _stats():
    a, p = C.c_int64(), C.c_int64()
    call("aic_hip_mem_stats", C.byref(a), C.byref(p))
    return a.value, p.value


def _alloc(n, s):
    p = C.c_void_p()
    call("aic_hip_mem_alloc_async", C.byref(p), n, s)
    return p.value


def test_allocator_stats_round_trip_and_reuse():
    s = torch.cuda.Stream()
    sp = s.cuda_stream
    a0, p0 = _stats()
    sizes = [1, 4096, 3 << 20, 100_000_007]
    ptrs = [_alloc(n, sp) for n in sizes]
    assert all(p and p % 256 == 0 for p in ptrs) and len(set(ptrs)) == len(ptrs)
    a1, p1 = _stats()
    assert a1 - a0 == sum(sizes) and p1 >= a0 + sum(sizes)
    # the memory is usable on its stream: write a pattern, read it back through memcpy_sync
    host = np.arange(sizes[2] // 4, dtype=np.int32)
    call("aic_hip_memcpy_sync", ptrs[2], host.ctypes.data, sizes[2], sp)
    back = np.empty_like(host)
    call("aic_hip_memcpy_sync", back.ctypes.data, ptrs[2], sizes[2], sp)
    np.testing.assert_array_equal(back, host)
    for p in ptrs:
        call("aic_hip_mem_free_async", p, sp)
    a2, p2 = _stats()
    assert a2 == a0 and p2 == p1  # the high-water mark stays
    # freed blocks stay cached in the pool: an allocation of a freed size succeeds on the same stream
    q = _alloc(sizes[3], sp)
    call("aic_hip_mem_free_async", q, sp)
    s.synchronize()
    # zero bytes is a null pointer and a no-op free
    assert _alloc(0, sp) is None
    call("aic_hip_mem_free_async", None, sp)


def test_allocator_rejects_foreign_pointer():
    sp = torch.cuda.current_stream().cuda_stream
    t = torch.empty(16, device="cuda")
    a0, _ = _stats()
    with pytest.raises(_lib.AicError) as e:
        call("aic_hip_mem_free_async", t.data_ptr(), sp)  # not from the pool: refused on the host
    assert e.value.code == 1 and "did not allocate" in str(e.value)
    assert _stats()[0] == a0


def test_memcpy_sync_device_to_device_and_empty():
    a = torch.arange(1000, dtype=torch.float32, device="cuda")
    b = torch.zeros_like(a)
    sp = torch.cuda.current_stream().cuda_stream
    call("aic_hip_memcpy_sync", b.data_ptr(), a.data_ptr(), 4000, sp)
    assert torch.equal(a, b)
    call("aic_hip_memcpy_sync", None, None, 0, sp)
    with pytest.raises(_lib.AicError):
        call("aic_hip_memcpy_sync", None, a.data_ptr(), 4, sp)
