"""The loader's device path: batches gathered in HBM (resident corpus) and batches streamed
through pinned buffers equal the host batches of an identical loader, across an epoch
boundary and a partial last batch; a training step fed from device batches equals the step
fed the same batch from host memory."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

import autonomousaicore_amd as aic  # noqa: E402
from autonomousaicore_amd.data import BinaryTokenDataset, DataLoader  # noqa: E402
from tests.test_gpu_step import TINY, build, make_params  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)


@pytest.mark.parametrize("resident", [True, False])
def test_device_batches_equal_host_batches(tmp_path, resident):
    rng = np.random.default_rng(3)
    p = str(tmp_path / "t.bin")
    BinaryTokenDataset.write_binary_file(p, rng.integers(0, 32000, 70001))
    ds = BinaryTokenDataset(p, seq_len=512, stride=384)
    host = DataLoader(ds, batch_size=16, shuffle=True, seed=5)
    dev = DataLoader(ds, batch_size=16, shuffle=True, seed=5, device="cuda", resident=resident)
    assert host.num_batches() == dev.num_batches() == (ds.size() + 15) // 16
    for epoch in range(2):
        n = 0
        while host.has_next():
            hx, hy = host.next()
            dx, dy = dev.next()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(dx.cpu().numpy(), hx)
            np.testing.assert_array_equal(dy.cpu().numpy(), hy)
            n += hx.shape[0]
        assert n == ds.size() and not dev.has_next()
        host.reset()
        dev.reset()


def test_training_from_device_batches():
    B, S = 8, 64
    rng = np.random.default_rng(9)
    ds = BinaryTokenDataset(rng.integers(0, TINY["vocab"], 20000), seq_len=S)
    loader = DataLoader(ds, batch_size=B, shuffle=True, seed=42, device="cuda")
    ref = DataLoader(ds, batch_size=B, shuffle=True, seed=42)
    a, b = build(TINY), build(TINY)
    params = make_params(a, 77)
    a.set_params(params)
    b.set_params(params)
    for _ in range(3):
        x, y = loader.next()
        torch.cuda.synchronize()
        hx, hy = ref.next()
        sa = a.train_step(x.data_ptr(), y.data_ptr(), B, S)
        sb = b.train_step(hx, hy, B, S)
        assert sa.loss == sb.loss
    np.testing.assert_array_equal(a.get_params(), b.get_params())
    a.close()
    b.close()
