"""Token data for the training step, mirroring the reference's data API
(aic::data::BinaryTokenDataset and DataLoader, include/data/dataset.hpp and
include/data/dataloader.hpp).  All work happens in libaic_hip.so: the dataset maps the
int64 token file, the loader keeps the reference's sample order (std::shuffle over
std::mt19937_64(seed)) and writes batches either to host arrays or to device buffers
(HBM-resident corpus + one gather kernel per batch, or pinned double-buffered copies)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


class BinaryTokenDataset:
    """BinaryTokenDataset(path or int64 tokens, seq_len, stride=0)."""

    def __init__(self, source, seq_len: int, stride: int = 0):
        h = C.c_void_p()
        if isinstance(source, (str, bytes)):
            path = source.encode() if isinstance(source, str) else source
            _lib.call("aic_dataset_open", path, seq_len, stride, C.byref(h))
        else:
            t = np.ascontiguousarray(source, np.int64)
            _lib.call("aic_dataset_from_tokens", t.ctypes.data, t.size, seq_len, stride, C.byref(h))
        self._h = h
        self.seq_len = seq_len

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.call("aic_dataset_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def size(self) -> int:
        return int(_lib.load().aic_dataset_size(self._h))

    __len__ = size

    def total_tokens(self) -> int:
        return int(_lib.load().aic_dataset_total_tokens(self._h))

    def get_item(self, idx: int):
        x = np.empty(self.seq_len, np.int64)
        y = np.empty(self.seq_len, np.int64)
        _lib.call("aic_dataset_get_item", self._h, idx, x.ctypes.data, y.ctypes.data)
        return x, y

    @staticmethod
    def write_binary_file(path: str, tokens) -> None:
        t = np.ascontiguousarray(tokens, np.int64)
        _lib.call("aic_dataset_write_binary_file", path.encode(), t.ctypes.data, t.size)


class DataLoader:
    """DataLoader(dataset, batch_size, shuffle=False, drop_last=False, device="cpu", seed=42).
    On "cuda" next() returns torch int64 tensors on the current device, written on the current
    stream; resident=True keeps the whole token array in HBM and gathers batches there."""

    def __init__(self, dataset: BinaryTokenDataset, batch_size: int, shuffle: bool = False, drop_last: bool = False,
                 device: str = "cpu", seed: int = 42, resident: bool = True):
        h = C.c_void_p()
        _lib.call("aic_loader_create", dataset._h, batch_size, 1 if shuffle else 0, 1 if drop_last else 0,
                  C.c_uint64(seed), 1 if resident else 0, C.byref(h))
        self._h = h
        self._ds = dataset
        self.batch_size = batch_size
        self.device = device

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.call("aic_loader_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def num_batches(self) -> int:
        return int(_lib.load().aic_loader_num_batches(self._h))

    def has_next(self) -> bool:
        return bool(_lib.load().aic_loader_has_next(self._h))

    def reset(self) -> None:
        _lib.call("aic_loader_reset", self._h)

    def next(self):
        S = self._ds.seq_len
        b = C.c_int64()
        if self.device == "cpu":
            x = np.empty((self.batch_size, S), np.int64)
            y = np.empty((self.batch_size, S), np.int64)
            _lib.call("aic_loader_next_host", self._h, x.ctypes.data, y.ctypes.data, C.byref(b))
            return x[:b.value], y[:b.value]
        import torch
        x = torch.empty((self.batch_size, S), dtype=torch.int64, device=self.device)
        y = torch.empty_like(x)
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.call("aic_loader_next_device", self._h, x.data_ptr(), y.data_ptr(), C.byref(b), C.c_void_p(stream))
        return x[:b.value], y[:b.value]

    def __iter__(self):
        while self.has_next():
            yield self.next()
