"""The C ABI from a C program (no GPU needed): include/fa_mi355x.h compiles as
C99 and as C++17 with every warning an error, and a program linked against
libfa_mi355x.so calls it the way the reference's C++ engine would
(scripts/deepseek_native_engine.sh calls its kernels from C++ host code):
the ABI version, the workspace sizing of the paged and token-major entries,
and an argument rejected with its status code and fa_last_error message.
The values must equal what the same calls return through ctypes."""
import os
import shutil
import subprocess

import pytest

from hrm_flashrenderer_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")

PROGRAM = r"""
#include <stdio.h>
#include "fa_mi355x.h"

int main(void) {
  printf("version %d\n", fa_abi_version());
  printf("paged %zu\n", fa_paged_workspace_bytes(64, 64, 1, 128, 8, 1025, 16, 8));
  printf("token_major %zu\n", fa_decode_token_major_workspace_bytes(40, 8, 128, 32767, 5));
  /* head_dim 96 is rejected before any device work (pointers never read) */
  int dummy = 0;
  int rc = fa_flash_attn_fwd(&dummy, &dummy, &dummy, &dummy, FA_DTYPE_F16, 1, 8, 8, 16, 16, 96,
                             1, 0, 0, NULL, NULL, NULL);
  printf("rc %d\n", rc);
  printf("msg %s\n", fa_last_error());
  return rc == FA_ERR_INVALID ? 0 : 1;
}
"""


def _compiler(name):
    path = shutil.which(name)
    if path is None:
        pytest.skip(f"{name} not installed")
    return path


@pytest.mark.parametrize("cc,std,suffix", [("gcc", "-std=c99", ".c"), ("g++", "-std=c++17", ".cpp")])
def test_header_compiles_cleanly(tmp_path, cc, std, suffix):
    src = tmp_path / ("h" + suffix)
    src.write_text('#include "fa_mi355x.h"\nint main(void) { return fa_abi_version() < 0; }\n')
    subprocess.run([_compiler(cc), std, "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", INCLUDE,
                    "-c", str(src), "-o", str(tmp_path / "h.o")], check=True)


def test_c_program_calls_the_library(tmp_path):
    lib_path = _lib.LIB_PATH
    if not os.path.exists(lib_path):
        pytest.skip("library not built")
    src = tmp_path / "prog.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "prog"
    libdir = os.path.dirname(lib_path)
    libname = os.path.basename(lib_path)
    subprocess.run([_compiler("gcc"), "-std=c99", "-Wall", "-Werror", "-I", INCLUDE, str(src),
                    "-o", str(exe), os.path.join(libdir, libname), "-Wl,-rpath," + libdir],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True,
                         timeout=120).stdout
    got = dict(line.split(" ", 1) for line in out.strip().splitlines())
    lib = _lib.load()
    assert int(got["version"]) == lib.fa_abi_version() == _lib.FA_ABI_VERSION
    assert int(got["paged"]) == lib.fa_paged_workspace_bytes(64, 64, 1, 128, 8, 1025, 16, 8) > 0
    assert int(got["token_major"]) == lib.fa_decode_token_major_workspace_bytes(
        40, 8, 128, 32767, 5) > 0
    assert int(got["rc"]) == -1
    assert got["msg"] == "Supported head_dim: 64 or 128"
