"""The boundary seen from C, as the reference's own (C) host would see it:

* include/rmda_moe.h is valid C17 (gcc -std=c17 -pedantic -Werror), every
  function it declares links against librmda_moe.so, and the program loads;
* the argument structs have the size, field offsets and field types of the
  reference's push-constant structs in src/pc.h, checked with _Static_assert
  against the reference tree's own header (skipped where that tree is absent).
"""
import os
import subprocess

import pytest

from rmda_moe import _lib

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
INC = os.path.join(REPO, "include")
CSRC = os.path.join(REPO, "r-mda_amd", "csrc")
REF_PC_H = "/root/reference/src/pc.h"


def gcc(args, cwd):
    r = subprocess.run(["gcc"] + args, cwd=cwd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]


def test_header_is_c17_and_links(tmp_path):
    names = _lib.header_functions()
    assert len(names) > 30
    src = ["#include <stdio.h>", "#include \"rmda_moe.h\"", "",
           "static void (*const every[])(void) = {"]
    src += ["    (void (*)(void))%s," % n for n in names]
    src += ["};", "", "int main(void) {",
            "    printf(\"%u %s\\n\", (unsigned)(sizeof(every) / sizeof(every[0])), rmda_moe_version());",
            "    return 0;", "}", ""]
    (tmp_path / "every.c").write_text("\n".join(src))
    lib = os.path.join(CSRC, "librmda_moe.so")
    if not os.path.exists(lib):
        pytest.skip("librmda_moe.so not built")
    gcc(["-std=c17", "-pedantic", "-Wall", "-Wextra", "-Werror", "-I", INC, "-o", "every", "every.c",
         "-L", CSRC, "-lrmda_moe", "-Wl,-rpath," + CSRC, "-Wl,-rpath-link,/opt/rocm/lib"], tmp_path)
    r = subprocess.run([str(tmp_path / "every")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split()[0] == str(len(names))


@pytest.mark.skipif(not os.path.exists(REF_PC_H), reason="reference tree absent")
def test_structs_match_reference_pc_h(tmp_path):
    gcc(["-std=c17", "-Wall", "-Wextra", "-Werror", "-I", INC, "-I", os.path.dirname(REF_PC_H), "-c",
         os.path.join(HERE, "c", "abi_layout.c"), "-o", str(tmp_path / "abi_layout.o")], tmp_path)
