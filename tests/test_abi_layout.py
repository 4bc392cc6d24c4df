"""The ctypes records of adafactor8bit._native against the C structs of
include/adafactor8bit_amd.h.

Every Structure whose docstring says "Mirror of ``name``" must have the C struct's
size and each of its fields at the C offset: a program compiled with the host C
compiler against the header prints sizeof and offsetof for the mirror's field
names (a name the struct lacks fails the compile).  A record that drifted from
the header would hand the kernels shifted pointers.
"""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _mirrors():
    from adafactor8bit import _native as nat
    out = []
    for name in dir(nat):
        cls = getattr(nat, name)
        if isinstance(cls, type) and issubclass(cls, ctypes.Structure) and cls.__doc__:
            m = re.search(r"Mirror of ``(\w+)``", cls.__doc__)
            if m:
                out.append((m.group(1), cls))
    return sorted(out, key=lambda x: x[0])


def test_every_mirror_matches_the_header(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    mirrors = _mirrors()
    assert len(mirrors) >= 8
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "adafactor8bit_amd.h"', "int main(void) {"]
    for cname, cls in mirrors:
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for f in cls._fields_:
            lines.append(f'  printf("{cname} {f[0]} %zu\\n", offsetof({cname}, {f[0]}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, cls in mirrors:
        assert ctypes.sizeof(cls) == got[(cname, "sizeof")], f"{cname}: sizeof"
        for f in cls._fields_:
            assert getattr(cls, f[0]).offset == got[(cname, f[0])], f"{cname}.{f[0]}: offset"
