"""include/anedvd_moe.h as a C consumer sees it (Zig's @cImport translates it as C):
a strict C99 program includes the header, links the library and calls through it
without a GPU (the ABI version, the last-error string, and a refused call)."""
import os
import shutil
import subprocess

import pytest

from anedvd_amd import moe
from tests.conftest import ROOT

PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "anedvd_moe.h"

int main(void) {
    anedvd_moe_stats st;
    anedvd_moe_layer_desc desc;
    anedvd_gguf_moe_cfg cfg;
    int rc;
    memset(&st, 0, sizeof st);
    memset(&desc, 0, sizeof desc);
    if (anedvd_moe_abi_version() != ANEDVD_MOE_ABI_VERSION) return 1;
    /* a host-only call that is refused: no GGUF magic in 4 zero bytes */
    rc = anedvd_gguf_moe_info("\0\0\0\0", 4, 0, &cfg);
    if (rc != ANEDVD_E_NOT_GGUF && rc != ANEDVD_E_TRUNCATED) return 2;
    if (anedvd_moe_last_error() == NULL || strlen(anedvd_moe_last_error()) == 0) return 3;
    printf("abi %d sizeof(stats) %u sizeof(desc) %u rc %d\n", anedvd_moe_abi_version(), (unsigned)sizeof st,
           (unsigned)sizeof desc, rc);
    return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_header_compiles_as_c99_and_links(tmp_path):
    src = tmp_path / "use_abi.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "use_abi"
    libdir = os.path.dirname(moe.LIB_PATH)
    cmd = ["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           str(src), "-o", str(exe), moe.LIB_PATH, "-Wl,-rpath," + libdir]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    assert run.stdout.startswith("abi %d" % moe.lib().anedvd_moe_abi_version())
