"""Device buffers owned through the library's C ABI.

The reference's trainer owns every device buffer it trains from (the
rollout's observations, actions, log-probs, values, rewards, terminals and
the replay scratch; pufferlib.cu:2616-2674).  The host mirror does the same
here through ``ptcg_device_alloc`` / ``ptcg_memcpy``, so the product path
needs no other GPU runtime.  A :class:`DeviceArray` is a typed, shaped,
contiguous device allocation freed when the object goes away; kernels get
its address from :meth:`DeviceArray.data_ptr`.
"""
import ctypes

import numpy as np

from .native import lib, check, c_void_p

H2D, D2H, D2D = 0, 1, 2


class DeviceArray:
    """Contiguous device array of ``shape`` and numpy ``dtype`` (zero-filled
    at allocation)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(x) for x in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        self._p = c_void_p()
        check(lib().ptcg_device_alloc(self.nbytes, ctypes.byref(self._p)))

    @classmethod
    def from_numpy(cls, a, dtype=None):
        a = np.ascontiguousarray(a, dtype=dtype if dtype is not None else None)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    def data_ptr(self):
        return self._p.value or 0

    def numel(self):
        return self.size

    def __len__(self):
        return self.shape[0] if self.shape else 1

    def upload(self, a, stream=None):
        """Host array of the same byte size into this buffer (synchronous)."""
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise RuntimeError(f"upload: {a.nbytes} bytes into a {self.nbytes}-byte device array")
        check(lib().ptcg_memcpy(self._p, a.ctypes.data, self.nbytes, H2D, stream))

    def copy_(self, src, stream=None):
        """Device-to-device copy of another array of the same byte size,
        ordered on ``stream`` (an object with data_ptr(), or a DeviceArray)."""
        nb = src.nbytes if isinstance(src, DeviceArray) else src.numel() * src.element_size()
        if nb != self.nbytes:
            raise RuntimeError(f"copy_: {nb} bytes into a {self.nbytes}-byte device array")
        check(lib().ptcg_memcpy(self._p, c_void_p(src.data_ptr()), self.nbytes, D2D, stream))
        return self

    def numpy(self, stream=None):
        """Host copy (waits for ``stream`` first)."""
        out = np.empty(self.shape, self.dtype)
        check(lib().ptcg_memcpy(out.ctypes.data, self._p, self.nbytes, D2H, stream))
        return out

    def item(self):
        if self.size != 1:
            raise RuntimeError(f"item: array of {self.size} elements")
        return self.numpy().reshape(-1)[0].item()

    def clone(self):
        d = DeviceArray(self.shape, self.dtype)
        d.copy_(self)
        return d

    def free(self):
        if self._p.value:
            check(lib().ptcg_device_free(self._p))
            self._p = c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self):
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype.name}, ptr=0x{self.data_ptr():x})"


def empty(shape, dtype=np.float32):
    return DeviceArray(shape, dtype)


def device_count():
    n = ctypes.c_int()
    check(lib().ptcg_device_count(ctypes.byref(n)))
    return n.value


def synchronize():
    check(lib().ptcg_device_synchronize())


class Event:
    """A timing event on the library's device (hipEvent_t)."""

    def __init__(self):
        self._e = c_void_p()
        check(lib().ptcg_event_create(ctypes.byref(self._e)))

    def record(self, stream=None):
        check(lib().ptcg_event_record(self._e, stream))

    def elapsed_ms(self, end):
        """Milliseconds from this event to ``end`` (waits for ``end``)."""
        ms = ctypes.c_float()
        check(lib().ptcg_event_elapsed_ms(self._e, end._e, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self._e.value:
                check(lib().ptcg_event_destroy(self._e))
                self._e = c_void_p()
        except Exception:
            pass
