"""Device memory for callers of the CIH_IO_DEVICE forward, through
libamdhip64 directly (no torch): allocate, copy, free.  The forward itself
never needs this module; it is the plumbing a caller that keeps tokens and
outputs in HBM (the benchmark, the device-I/O tests) uses.
"""
import ctypes

H2D, D2H, D2D = 1, 2, 3


class Hip:
    """Minimal device-memory plumbing through libamdhip64."""

    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so")
        self.L.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.L.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.L.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
        self.L.hipFree.argtypes = [ctypes.c_void_p]

    def malloc(self, n):
        p = ctypes.c_void_p()
        if self.L.hipMalloc(ctypes.byref(p), max(int(n), 1)) != 0:
            raise RuntimeError("hipMalloc failed")
        return p.value

    def h2d(self, dst, arr):
        if self.L.hipMemcpy(ctypes.c_void_p(dst), arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes, H2D) != 0:
            raise RuntimeError("hipMemcpy H2D failed")

    def d2h(self, arr, src):
        if self.L.hipMemcpy(arr.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(src), arr.nbytes, D2H) != 0:
            raise RuntimeError("hipMemcpy D2H failed")

    def d2d(self, dst, src, nbytes):
        if self.L.hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes, D2D) != 0:
            raise RuntimeError("hipMemcpy D2D failed")

    def memset(self, dst, value, nbytes):
        if self.L.hipMemset(ctypes.c_void_p(dst), value, nbytes) != 0:
            raise RuntimeError("hipMemset failed")

    def sync(self):
        self.L.hipDeviceSynchronize()

    def free(self, p):
        self.L.hipFree(ctypes.c_void_p(p))
