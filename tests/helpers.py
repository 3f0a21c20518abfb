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


_HIP = None


def hip_runtime():
    """The HIP runtime libneedle_hip.so itself links, through ctypes."""
    global _HIP
    if _HIP is None:
        import ctypes as C

        lib = C.CDLL("libamdhip64.so.7")
        lib.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        lib.hipFree.argtypes = [C.c_void_p]
        lib.hipDeviceSynchronize.argtypes = []
        _HIP = lib
    return _HIP


def read_device(ptr, shape, dtype):
    """A host copy of `shape` elements of `dtype` at device address ptr."""
    out = np.empty(shape, dtype)
    lib = hip_runtime()
    assert lib.hipDeviceSynchronize() == 0
    assert lib.hipMemcpy(out.ctypes.data, ptr, out.nbytes, 2) == 0
    return out


class DeviceArray:
    """A host array copied into HBM with the HIP runtime libneedle_hip.so
    itself links (hipMalloc / hipMemcpy), for the entry points that take
    device pointers; `.ptr` is the device address, `.read()` copies back."""

    _hip = None

    def __init__(self, host):
        import ctypes as C

        DeviceArray._hip = hip_runtime()
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


def kv_quotients(raw):
    """x / s for every element of K/V vectors raw [..., 64] with the
    reference's float64 arithmetic: s = max(1e-12, max|x|) / 127 per vector
    (model/runtime.ts:697-714), the quotient its roundTiesToEven rounds."""
    x = np.asarray(raw, dtype=np.float64)
    m = np.maximum(1e-12, np.abs(x).max(axis=-1, keepdims=True))
    return x / (m / 127)


def assert_codes_or_boundary_flips(got, want, raw, delta, what=""):
    """int8 codes equal the oracle's, or are one apart with the oracle's exact
    quotient x / s within `delta` of the half-integer between the two codes
    (the value sat on a rounding boundary and an input that differs in its
    last bits rounded the other way).  A wrong quantizer, a wrong scale or a
    wrong slot would put differing codes anywhere in [0, 0.5) from the
    boundary.  Returns (number of differing codes, largest distance)."""
    got = np.asarray(got).astype(np.int64)
    want = np.asarray(want).astype(np.int64)
    differ = got != want
    if not differ.any():
        return 0, 0.0
    gap = np.abs(got - want)[differ].max()
    assert gap == 1, f"{what}: codes {int(gap)} apart"
    dist = np.abs(kv_quotients(raw) - (np.minimum(got, want) + 0.5))[differ]
    worst = float(dist.max())
    assert worst <= delta, (f"{what}: {int(differ.sum())} codes differ, one {worst:.3e} from "
                            f"the rounding boundary (bar {delta:.0e})")
    return int(differ.sum()), worst


def storekv_of_projections(proj, heads, kv_heads, k_norm, theta, positions):
    """#storeKV of a backend's own last-layer projections proj [M][q|k|v]
    with the oracle's arithmetic: per row m and KV head h the key is
    rmsNormSlice(k, k_norm) rotated at positions[m] (model/runtime.ts:
    479-500), the value the raw projection.  Returns the float32 vectors and
    the oracle's codes and scales: (k, v, k_codes, k_scales, v_codes,
    v_scales), vectors [M][kv_heads][64]."""
    import oracle

    proj = np.asarray(proj, dtype=np.float32)
    M = proj.shape[0]
    k = np.empty((M, kv_heads, 64), np.float32)
    v = proj[:, (heads + kv_heads) * 64:].reshape(M, kv_heads, 64).copy()
    kc = np.empty((M, kv_heads, 64), np.int8)
    vc = np.empty_like(kc)
    ks = np.empty((M, kv_heads), np.float32)
    vs = np.empty_like(ks)
    for m in range(M):
        for h in range(kv_heads):
            kh = proj[m, (heads + h) * 64:(heads + h + 1) * 64]
            k[m, h] = oracle.rope(oracle.rms_norm(kh, k_norm), 1, 64, int(positions[m]), theta)
            kc[m, h], ks[m, h] = oracle.kv_quantize(k[m, h])
            vc[m, h], vs[m, h] = oracle.kv_quantize(v[m, h])
    return k, v, kc, ks, vc, vs
