"""GPU presence probe shared by the tests (counts devices without creating a context)."""
import ctypes


def gpu_available() -> bool:
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        n = ctypes.c_int(0)
        return hip.hipGetDeviceCount(ctypes.byref(n)) == 0 and n.value > 0
    except OSError:
        return False
