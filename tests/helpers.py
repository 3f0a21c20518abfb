"""Assertion helpers shared by the test modules."""

import numpy as np


def assert_close(actual, expected, rtol=1e-3, atol=1e-4, what=""):
    """The fp32 parity bar: |a - e| <= atol + rtol * |e| elementwise."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    err = np.abs(actual - expected)
    bound = atol + rtol * np.abs(expected)
    bad = ~(err <= bound)
    if bad.any():
        i = int(np.flatnonzero(bad.reshape(-1))[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside rtol={rtol} atol={atol}; first at flat "
            f"index {i}: got {actual.reshape(-1)[i]!r}, want {expected.reshape(-1)[i]!r}; "
            f"max abs err {float(err.max()):.3e}")


class DeviceArray:
    """A host array copied into HBM with the HIP runtime libneedle_hip.so
    itself links (hipMalloc / hipMemcpy), for the entry points that take
    device pointers; `.ptr` is the device address, `.read()` copies back."""

    _hip = None

    def __init__(self, host):
        import ctypes as C

        if DeviceArray._hip is None:
            lib = C.CDLL("libamdhip64.so.7")
            lib.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
            lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
            lib.hipFree.argtypes = [C.c_void_p]
            lib.hipDeviceSynchronize.argtypes = []
            DeviceArray._hip = lib
        self.host = np.ascontiguousarray(host)
        self._c = C
        p = C.c_void_p()
        assert DeviceArray._hip.hipMalloc(C.byref(p), max(1, self.host.nbytes)) == 0
        self.ptr = p
        assert DeviceArray._hip.hipMemcpy(p, self.host.ctypes.data, self.host.nbytes, 1) == 0

    def read(self):
        out = np.empty_like(self.host)
        assert DeviceArray._hip.hipDeviceSynchronize() == 0
        assert DeviceArray._hip.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, 2) == 0
        return out

    def free(self):
        if self.ptr is not None:
            DeviceArray._hip.hipFree(self.ptr)
            self.ptr = None
