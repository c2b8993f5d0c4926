"""The C-ABI library loads and exports every symbol include/*.h declares
(no compute calls: this runs without a GPU)."""
from __future__ import annotations

import ctypes
import glob
import os
import re

from tensormark_amd import sampler

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(tms_\w+)\s*\(", src, re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = sampler.load_library()
    decl = declared_functions()
    assert "tms_sample_batch" in decl and "tms_create" in decl
    for name in decl:
        assert hasattr(lib, name), name
    assert set(decl) == set(sampler.EXPORTS)


def test_abi_version_and_struct_sizes():
    lib = sampler.load_library()
    assert lib.tms_abi_version() == 2
    assert ctypes.sizeof(sampler.SampleArgs) == 136
    assert ctypes.sizeof(sampler.RowParams) == 56
    assert lib.tms_status_string(-2).decode().startswith("batch")


def test_invalid_arguments_rejected_without_device_work():
    lib = sampler.load_library()
    assert lib.tms_sample_batch(None, None, None) == -1
    assert lib.tms_destroy(None) == -1
    h = ctypes.c_void_p()
    assert lib.tms_create(0, 0, 100, ctypes.byref(h)) == -1
    assert lib.tms_create(0, 1, 1 << 30, ctypes.byref(h)) == -1
