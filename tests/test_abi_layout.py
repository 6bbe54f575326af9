"""The ctypes mirrors of the C-ABI structs (kernel/_ext.py) match
include/saf_attn.h field by field: a C program built from the header prints
sizeof and offsetof of every field, compared with the ctypes layout.  A
field added to one side only would shift every field after it and make the
library read garbage, so this runs on the CPU with the rest of the host
tests."""
import ctypes
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _c_layout(tmp_path, struct, fields):
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "saf_attn.h"', "int main(void) {",
             f'  printf("{{\\"__sizeof\\": %zu", sizeof({struct}));']
    for f in fields:
        lines.append(f'  printf(", \\"{f}\\": %zu", offsetof({struct}, {f}));')
    lines += ['  printf("}\\n");', "  return 0;", "}"]
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    return json.loads(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
@pytest.mark.parametrize("cname,pyname", [("saf_tensor_t", "SafTensor"), ("saf_mixed_attn_args", "SafMixedAttnArgs")])
def test_ctypes_structs_match_header(tmp_path, cname, pyname):
    from kernel import _ext
    cls = getattr(_ext, pyname)
    names = [f[0] for f in cls._fields_]
    c = _c_layout(tmp_path, cname, names)
    assert c["__sizeof"] == ctypes.sizeof(cls), (cname, c["__sizeof"], ctypes.sizeof(cls))
    for n in names:
        assert c[n] == getattr(cls, n).offset, (cname, n, c[n], getattr(cls, n).offset)
