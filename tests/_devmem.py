"""Device buffers for the shared parity harness (tests/cpu/simt/run_parity.py) on a GPU: torch tensors
on cuda:0; every transfer synchronises the device, so the library's own stream has finished."""
import numpy as np
import torch


class TorchMem:
    """Harness buffers in device memory; transfers synchronise the device."""

    _types = {np.float32: torch.float32, np.int32: torch.int32, np.uint32: torch.int32}

    class Buf:
        def __init__(self, n, dtype):
            self.dtype = np.dtype(dtype)
            self.t = torch.zeros(n, dtype=TorchMem._types[self.dtype.type], device="cuda:0")
            self.ptr = self.t.data_ptr()

        def upload(self, x):
            a = np.ascontiguousarray(x, dtype=self.dtype)
            if self.dtype == np.uint32:
                a = a.view(np.int32)
            self.t.copy_(torch.from_numpy(a))
            torch.cuda.synchronize()

        def host(self):
            torch.cuda.synchronize()
            return self.t.cpu().numpy().view(self.dtype)

    def zeros(self, n, dtype):
        return self.Buf(n, dtype)


