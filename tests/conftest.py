"""Test configuration: the `gpu` marker, import paths, shared generators."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "oracle"), os.path.join(REPO, "esp32-needle-3_amd"),
          os.path.join(REPO, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def normal(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


@pytest.fixture
def rng():
    return np.random.default_rng(20261201)


# A device allocator for nda_set_allocator (the counterpart of the engine's
# ND_ALLOC / ND_FREE seams): hipMalloc / hipFree, refusing requests on demand,
# counting every request it sees.
ALLOC = C.CFUNCTYPE(C.c_void_p, C.c_size_t, C.c_void_p)
FREE = C.CFUNCTYPE(None, C.c_void_p, C.c_void_p)


class FailingAllocator:
    """hipMalloc / hipFree; refuses every request while `armed`, or only the
    n-th request counted from `refuse_nth` being set."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.hip.hipMalloc.restype = C.c_int
        self.hip.hipFree.argtypes = [C.c_void_p]
        self.hip.hipFree.restype = C.c_int
        self.armed = False
        self.refuse_nth = 0
        self.seen = 0
        self.refused = 0
        self._alloc = ALLOC(self.alloc)
        self._free = FREE(self.free)

    def alloc(self, nbytes, user):
        self.seen += 1
        if self.armed or (self.refuse_nth and self.seen == self.refuse_nth):
            self.refused += 1
            return None
        p = C.c_void_p()
        return p.value if self.hip.hipMalloc(C.byref(p), nbytes) == 0 else None

    def free(self, ptr, user):
        self.hip.hipFree(ptr)


@pytest.fixture
def allocator():
    import ndattn as N
    a = FailingAllocator()
    N._check(N.lib().nda_set_allocator(C.cast(a._alloc, C.c_void_p), C.cast(a._free, C.c_void_p), None))
    yield a
    a.armed = False
    a.refuse_nth = 0
    N._check(N.lib().nda_set_allocator(None, None, None))


