"""The C ABI: the library loads without a GPU and exports every declared symbol."""

import ctypes
import os
import re

import pytest

from conftest import ROOT


def test_header_declares_and_library_exports_everything():
    from cv3amd import _lib
    decls = _lib.parse_header()
    assert len(decls) > 40
    L = _lib.lib()
    for name in decls:
        assert hasattr(L, name), name


def test_every_exported_symbol_is_declared():
    from cv3amd import _lib
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (cv3_\w+)", out))
    assert exported == set(_lib.parse_header())


def test_error_codes_map_to_reference_exceptions():
    """A call that fails validation on the host side returns the mapped exception
    (no GPU involved: the argument check runs before any launch)."""
    from cv3amd import _lib
    with pytest.raises(ValueError):
        _lib.call("quantize_q8", None, 4, 0, 64, _lib.F16, None, None, None)
    with pytest.raises(ValueError):
        _lib.call("attention", None, None, None, None, 1, 14, 4, 1, 1, 64, None, None, None, None,
                  1.0, 0, 0, 0, None)
    assert "multiple" in _lib.lib().cv3_last_error().decode()


def test_no_cpu_fallback_in_the_package():
    """The shipped package never imports the oracle."""
    pkg = os.path.join(ROOT, "cosyvoice3-cpu_amd")
    for dp, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dp, f)).read()
                assert "import oracle" not in src and "from oracle" not in src, f


def test_init_as_the_first_library_call_does_not_deadlock():
    """``_lib.init()`` holds the module lock while its own call loads the library; as the
    first call of a fresh process it must return (or raise without a GPU), not block."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from cv3amd import _lib\n"
            "try:\n    _lib.init()\nexcept Exception as e:\n    print(type(e).__name__)\n"
            "print('returned')\n") % os.path.join(ROOT, "cosyvoice3-cpu_amd")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=60)
    assert "returned" in r.stdout, r.stdout + r.stderr
