"""``BatchFetcher``: prefetching batches of a host array onto the GPU.

Same constructor and ``next()`` as the reference's ``sdfoam.BatchFetcher``
(torch_bindings/torch_bindings.cpp:32-83, src/utils/batch_fetcher.cpp):
``BatchFetcher(data, batch_size, shuffle)`` over a CPU tensor ``data`` of
rows ``data[i]``; ``next()`` returns a new CUDA tensor
``[batch_size, *data.shape[1:]]`` holding the next batch -- random rows
(seeded per element exactly as the reference seeds them, so fetchers over
parallel arrays draw the same rows) or consecutive rows, wrapping around.

The work runs in libsdfoam_hip.so, in one of two ways:

* device-resident (the default when the array's rows are whole 32-bit words
  and it takes at most an eighth of the device's memory): the array is
  uploaded once at construction, and ``next()`` gathers the batch's rows on
  the GPU (``sdf_batch_gather``) on the current stream.  The reference keeps
  the array on the host; an MI355X holds a training set of tens of millions
  of rays many times over.  Later changes to the host tensor are not seen;
* streamed (``resident=False``, or rows of other sizes): a native worker
  thread gathers rows into pinned staging buffers and uploads them on its own
  stream into a ring of device slots (allocated here with torch); ``next()``
  queues the copy of the next slot on the current stream without waiting for
  the upload on the host.

Both give the same batches.
"""

from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import check


class BatchFetcher:
    def __init__(self, data: torch.Tensor, batch_size: int, shuffle: bool,
                 device=None, num_threads: int = 0, resident=None):
        if not isinstance(data, torch.Tensor):
            raise RuntimeError("data must be a torch.Tensor")
        if data.device.type != "cpu":
            raise RuntimeError("data must be a CPU tensor")
        if data.dim() < 1 or data.size(0) == 0:
            raise RuntimeError("data must have at least one row")
        batch_size = int(batch_size)
        if batch_size <= 0:
            raise RuntimeError("batch_size must be positive")
        self._data = data.contiguous()
        num_bytes = self._data.numel() * self._data.element_size()
        stride = num_bytes // self._data.size(0)
        self._shape = (batch_size,) + tuple(self._data.shape[1:])
        self._dtype = self._data.dtype
        self._device = torch.device("cuda", torch.cuda.current_device()) if device is None \
            else torch.device(device)
        self.batch_size = batch_size
        L = _lib.lib()
        self._handle = None
        if resident is None:
            total = torch.cuda.get_device_properties(self._device).total_memory
            resident = stride % 4 == 0 and num_bytes <= total // 8
        elif resident and stride % 4 != 0:
            raise RuntimeError("a device-resident BatchFetcher needs rows of whole 32-bit words")
        self.resident = bool(resident)
        if self.resident:
            with torch.cuda.device(self._device):
                self._device_data = self._data.to(self._device)
            self._num_rows = int(self._data.size(0))
            self._stride = int(stride)
            self._shuffle = bool(shuffle)
            self._batch = 0
            self._open = True
            return
        ring_bytes = int(L.sdf_batch_fetcher_ring_bytes(stride, batch_size))
        self._ring = torch.empty(ring_bytes, dtype=torch.uint8, device=self._device)
        handle = C.c_void_p()
        with torch.cuda.device(self._device):
            check(L.sdf_batch_fetcher_create(
                self._data.data_ptr(), num_bytes, stride, batch_size, 1 if shuffle else 0,
                self._ring.data_ptr(), ring_bytes, int(num_threads), C.byref(handle)))
        self._handle = handle

    def next(self) -> torch.Tensor:
        if self.resident:
            if not self._open:
                raise RuntimeError("BatchFetcher is closed")
            out = torch.empty(self._shape, dtype=self._dtype, device=self._device)
            with torch.cuda.device(self._device):
                check(_lib.lib().sdf_batch_gather(
                    self._device_data.data_ptr(), self._num_rows, self._stride,
                    self._batch & 0xFFFFFFFF, self.batch_size, 1 if self._shuffle else 0,
                    out.data_ptr(), _lib.stream_handle(self._device)))
            self._batch += 1
            return out
        if self._handle is None:
            raise RuntimeError("BatchFetcher is closed")
        out = torch.empty(self._shape, dtype=self._dtype, device=self._device)
        with torch.cuda.device(self._device):
            check(_lib.lib().sdf_batch_fetcher_next(self._handle, out.data_ptr(),
                                                    _lib.stream_handle(self._device)))
        return out

    def close(self) -> None:
        if getattr(self, "resident", False):
            self._open = False
            self._device_data = None
            return
        if getattr(self, "_handle", None) is not None:
            h, self._handle = self._handle, None
            check(_lib.lib().sdf_batch_fetcher_destroy(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def batch_rows(batch_index: int, batch_size: int, num_rows: int, shuffle: bool):
    """Row indices batch ``batch_index`` takes (host computation)."""
    import numpy as np

    out = np.zeros(batch_size, dtype=np.uint32)
    _lib.lib().sdf_batch_rows(batch_index, batch_size, num_rows, 1 if shuffle else 0,
                              out.ctypes.data_as(C.c_void_p))
    return out
