"""Token dataset and loader on the CPU: the reference's known answers
(tests/unit/test_data.cpp:63-146), the sample order against std::shuffle / std::mt19937_64
(tests/golden/shuffle_order.json, written by tests/golden/make_shuffle_golden.py), epochs
and drop_last."""
import json
import os

import numpy as np
import pytest

from autonomousaicore_amd import AicError
from autonomousaicore_amd.data import BinaryTokenDataset, DataLoader

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "shuffle_order.json")))


def test_in_memory_sliding_window():
    ds = BinaryTokenDataset(np.arange(100), seq_len=8, stride=4)
    assert ds.size() == 23                     # (100 - 1 - 8) / 4 + 1
    x0, y0 = ds.get_item(0)
    np.testing.assert_array_equal(x0, np.arange(8))
    np.testing.assert_array_equal(y0, np.arange(1, 9))
    x1, y1 = ds.get_item(1)
    np.testing.assert_array_equal(x1, np.arange(4, 12))
    np.testing.assert_array_equal(y1, np.arange(5, 13))
    with pytest.raises(AicError):
        ds.get_item(23)
    # stride 0 means seq_len; too few tokens give no sample
    assert BinaryTokenDataset(np.arange(100), 8).size() == (100 - 9) // 8 + 1
    assert BinaryTokenDataset(np.arange(8), 8).size() == 0
    assert BinaryTokenDataset(np.arange(9), 8).size() == 1


def test_memory_mapped_file(tmp_path):
    p = str(tmp_path / "tokens.bin")
    BinaryTokenDataset.write_binary_file(p, np.arange(500) * 2)
    assert os.path.getsize(p) == 500 * 8
    ds = BinaryTokenDataset(p, seq_len=16, stride=8)
    assert ds.total_tokens() == 500 and ds.size() == (500 - 17) // 8 + 1
    x, y = ds.get_item(0)
    np.testing.assert_array_equal(x, np.arange(16) * 2)
    np.testing.assert_array_equal(y, np.arange(1, 17) * 2)
    open(str(tmp_path / "bad.bin"), "wb").write(b"\0" * 12)
    with pytest.raises(AicError):
        BinaryTokenDataset(str(tmp_path / "bad.bin"), 4)
    with pytest.raises(AicError):
        BinaryTokenDataset(str(tmp_path / "missing.bin"), 4)


def samples_of(x, stride):
    return [int(v) // stride for v in x[:, 0]]


def test_batching_shuffling_and_drop_last():
    ds = BinaryTokenDataset(np.arange(120), seq_len=8, stride=4)
    assert ds.size() == 28
    loader = DataLoader(ds, batch_size=8, shuffle=True, drop_last=False)
    assert loader.num_batches() == 4
    sizes, order = [], []
    for x, y in loader:
        assert x.shape[1] == y.shape[1] == 8
        np.testing.assert_array_equal(y, x + 1)
        sizes.append(x.shape[0])
        order += samples_of(x, 4)
    assert sizes == [8, 8, 8, 4]
    assert order == GOLDEN["28_42"][0]                 # std::shuffle with std::mt19937_64(42)
    loader.reset()
    order2 = [s for x, _ in loader for s in samples_of(x, 4)]
    assert order2 == GOLDEN["28_42"][1]                # the second epoch: a second shuffle
    assert DataLoader(ds, batch_size=8, shuffle=False, drop_last=True).num_batches() == 3
    seq = [s for x, _ in DataLoader(ds, 8, shuffle=False, drop_last=True) for s in samples_of(x, 4)]
    assert seq == list(range(24))
    with pytest.raises(AicError):
        DataLoader(ds, 0)


@pytest.mark.parametrize("n,seed", [(23, 42), (1000, 7), (1, 42)])
def test_shuffle_order_matches_std_shuffle(n, seed):
    ds = BinaryTokenDataset(np.arange(n + 1), seq_len=1, stride=1)
    assert ds.size() == n
    loader = DataLoader(ds, batch_size=64, shuffle=True, seed=seed)
    for epoch in range(3):
        got = [int(v) for x, _ in loader for v in x[:, 0]]
        assert got == GOLDEN[f"{n}_{seed}"][epoch], epoch
        loader.reset()
