"""CPU check that every ctypes mirror of a C struct has the C layout.

The launchers and the backend table read these structs by offset: a mirror
that drifts from its header (a field added, moved or retyped on one side)
hands the GPU a wrong pointer.  A probe compiled from the headers prints each
field's offset and each struct's size; the mirrors must agree field for field.
"""
import ctypes
import os
import subprocess

import pytest

from igllm_amd import native
import launch_structs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# (C type, ctypes mirror): the mirror's field names are the C field names
MIRRORS = [
    ("igl_plane", native.Plane),
    ("igl_desk", native.Desk),
    ("igl_rng", native.Rng),
    ("igl_gemma_shape", native.GemmaShape),
    ("igl_code_view", launch_structs.CodeView),
    ("igl_gemv_prologue", launch_structs.Prologue),
]


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    work = tmp_path_factory.mktemp("layout")
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "igl_launch.h"', "int main(void) {"]
    for cname, mirror in MIRRORS:
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in mirror._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = work / "probe.c"
    src.write_text("\n".join(lines) + "\n")
    exe = work / "probe"
    subprocess.run(["gcc", "-std=c11", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "igllm_amd", "csrc"),
                    str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    table = {}
    for line in out.splitlines():
        cname, field, value = line.split()
        table[(cname, field)] = int(value)
    return table


@pytest.mark.parametrize("cname,mirror", MIRRORS, ids=[c for c, _ in MIRRORS])
def test_mirror_matches_header(c_layout, cname, mirror):
    assert ctypes.sizeof(mirror) == c_layout[(cname, "size")], cname
    for field, _ in mirror._fields_:
        assert getattr(mirror, field).offset == c_layout[(cname, field)], (cname, field)
