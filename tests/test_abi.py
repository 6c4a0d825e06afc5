"""The C ABI library loads and exports every function include/iam.h declares.
CPU only: nothing is called that needs a device."""
import ctypes as C
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol(iam):
    names = iam.header_symbols()
    assert len(names) > 40
    lib = iam.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_effort_quantile_matches_reference_kat(iam):
    # bucket_mul.hpp:164 computed on the host side of the library
    for e, target in {1.0: 4096, 0.5: 2049, 0.25: 1025, 0.125: 513, 0.05: 206}.items():
        assert 4096 - iam.effort_quantile(e) == target


def test_rope_table_host_function(iam, O):
    import numpy as np
    t = iam.rope_table(10000.0, 128, 32)
    assert np.array_equal(t.view(np.uint32), O.rope_table(10000.0, 128, 32).view(np.uint32))


def test_last_error_is_a_string(iam):
    assert isinstance(iam.last_error(), str)
    lib = iam.lib()
    rc = lib.iam_rope_table(C.c_double(10000.0), 127, 4, None)   # odd head_dim, null table
    assert rc == iam.IAM_E_INVALID
    assert "rope_table" in iam.last_error()
