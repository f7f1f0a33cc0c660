"""ctypes binding of libsnapjudge_fast_hip.so (snapjudge::FastSnapjudge over the
C ABI) for the tests: the reference's DecisionModel is loaded by the compiled
reference (oracle/_ref) and handed to the hook by pointer, as the reference's
Agent::accelerate (src/agent.cpp:363-386) hands its model."""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOOK_LIB = os.path.join(ROOT, "snapjudge_amd", "libsnapjudge_fast_hip.so")

# mangled names of the reference's declarations (include/snapjudge/fast.hpp:17-26)
REFERENCE_SYMBOLS = [
    "_ZN9snapjudge13FastSnapjudgeC1EPNS_13DecisionModelEib",
    "_ZN9snapjudge13FastSnapjudgeD1Ev",
    "_ZN9snapjudge13FastSnapjudge7forwardERKSt6vectorIS1_IlSaIlEESaIS3_EES7_S7_RKS1_IS1_IhSaIhEE"
    "SaIS9_EERKS3_RS1_IS1_IfSaIfEESaISH_EESK_",
]

_L = None


def lib():
    global _L
    if _L is None:
        import snapjudge_amd

        snapjudge_amd.lib()  # libsnapjudge_hip.so first (the hook's dependency)
        L = C.CDLL(HOOK_LIB)
        v = C.c_void_p
        L.sjfast_last_error.restype = C.c_char_p
        L.sjfast_create.argtypes = [v, C.c_int, C.c_int, C.c_int, C.c_int]
        L.sjfast_create.restype = v
        L.sjfast_destroy.argtypes = [v]
        L.sjfast_forward.argtypes = [v, v, v, v, v, v, C.c_int, C.c_int, C.c_int, v, v]
        L.sjfast_encode.argtypes = [v, v, v, C.c_int, C.c_int, v]
        _L = L
    return _L


class Fast:
    def __init__(self, model_ptr, max_len=0, graphs=True, precision=1, pad_rows=False):
        self.h = lib().sjfast_create(model_ptr, max_len, int(graphs), precision, int(pad_rows))
        if not self.h:
            raise RuntimeError(lib().sjfast_last_error().decode())

    def close(self):
        if self.h:
            lib().sjfast_destroy(self.h)
            self.h = None

    @staticmethod
    def _a(x):
        return x.ctypes.data_as(C.c_void_p)

    def forward(self, ids, mask, mp, mm, qt, n_act):
        ids, mask, mp, qt = (np.ascontiguousarray(x, np.int64) for x in (ids, mask, mp, qt))
        mm = np.ascontiguousarray(mm, np.uint8)
        N, L = ids.shape
        K = mp.shape[1]
        lg = np.empty((N, K), np.float32)
        act = np.empty((N, n_act), np.float32)
        rc = lib().sjfast_forward(self.h, self._a(ids), self._a(mask), self._a(mp), self._a(mm),
                                  self._a(qt), N, L, K, self._a(lg), self._a(act))
        if rc:
            raise RuntimeError(lib().sjfast_last_error().decode())
        return lg, act

    def encode(self, ids, mask, D):
        ids, mask = (np.ascontiguousarray(x, np.int64) for x in (ids, mask))
        N, L = ids.shape
        h = np.empty((N, L, D), np.float32)
        rc = lib().sjfast_encode(self.h, self._a(ids), self._a(mask), N, L, self._a(h))
        if rc:
            raise RuntimeError(lib().sjfast_last_error().decode())
        return h
