"""The reference-API hook (snapjudge::FastSnapjudge over the C ABI), CPU side:
it exports the reference's own FastSnapjudge symbols (so code compiled against
the reference's include/snapjudge/fast.hpp links to it) and rejects bad input
before touching the GPU."""
import ctypes as C
import os

import pytest

from hook_util import HOOK_LIB, REFERENCE_SYMBOLS

pytestmark = pytest.mark.skipif(not os.path.exists(HOOK_LIB),
                                reason="hook not built (needs the reference's headers)")


def test_exports_reference_fastsnapjudge_abi():
    L = C.CDLL(HOOK_LIB)
    for name in REFERENCE_SYMBOLS + ["sjfast_create", "sjfast_destroy", "sjfast_forward",
                                     "sjfast_encode", "sjfast_last_error"]:
        assert hasattr(L, name), name


def test_null_model_is_an_error_not_a_crash():
    from hook_util import lib

    assert lib().sjfast_create(None, 0, 1, 1, 0) is None
    assert b"null DecisionModel" in lib().sjfast_last_error()
